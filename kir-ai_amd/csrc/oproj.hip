// Output projection after attention: out[i][r] = sum_c W[r][c] * x[i][c], with
// W bf16 [rows][cols] row-major (an o_proj weight) and x the attention output
// of i = 0..n-1 sequences.  The reference computes this per sequence on the
// CPU (bf16_dot_f32_scalar, crates/llm-backend/src/core/safetensors/math.rs:66-72)
// or as a Metal matvec after its attention kernels
// (crates/llm-native-runtime/src/native_matvec.rs:4418-4492).
//
// On gfx950 it is a skinny GEMM on MFMA: out^T = W x^T.  A workgroup owns 32
// weight rows and 32 inputs; its 8 wavefronts split K, each running
// v_mfma_f32_32x32x16_bf16 with A = W (lane: row lane%32) and B = x^T (lane:
// input lane%32), then the 8 partial tiles are summed through LDS.  The order of
// K inside a wavefront is permuted so that every lane streams one contiguous
// half of its K slice (A and B use the same permutation, so the contraction is
// unchanged): step s, lane half h covers k = k0 + h * K/16 + 8s .. +8.
//
// A skinny projection has few 32 x 32 output tiles (o_proj of Qwen3-0.6B at
// B = 32: 32 tiles), too few workgroups to pull W from HBM at full rate.  Such
// calls also split K over `ksplit` workgroups per tile (grid z), each writing
// its partial tile to a workspace, and a second launch sums the partials in a
// fixed order (the result does not depend on scheduling).
#include "llh_internal.h"

namespace llh {

namespace {

constexpr int kWaves = kMatvecWaves;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)a, (__bf16)b});  // round to nearest even
}

template <typename XT>
__device__ __forceinline__ u32x4_t load_x8(const XT *p) {
  if constexpr (sizeof(XT) == 2) {
    return *reinterpret_cast<const u32x4_t *>(p);
  } else {
    const f32x4_t lo = *reinterpret_cast<const f32x4_t *>(p);
    const f32x4_t hi = *reinterpret_cast<const f32x4_t *>(p + 4);
    return u32x4_t{pack2(lo[0], lo[1]), pack2(lo[2], lo[3]), pack2(hi[0], hi[1]), pack2(hi[2], hi[3])};
  }
}

template <typename XT>
__global__ __launch_bounds__(64 * kWaves) void matvec_bf16_kernel(const MatvecArgs a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31;
  const int h = lane >> 5;
  const int r0 = blockIdx.x * 32;
  const int i0 = blockIdx.y * 32;
  const int kslice = a.cols / (int)gridDim.z;  // this workgroup's K slice
  const int kw = kslice / kWaves;               // this wavefront's
  const int kh = kw / 2;                        // per lane half
  const int k0 = (int)blockIdx.z * kslice + wave * kw + h * kh;
  const int row = min(r0 + c, a.rows - 1);  // rows / inputs past the end are computed on clamped data, not stored
  const int inp = min(i0 + c, a.n - 1);
  const uint16_t *wp = a.w + (size_t)row * a.cols + k0;
  const XT *xp = reinterpret_cast<const XT *>(a.x) + (size_t)inp * a.ldx + k0;

  f32x16_t acc;
#pragma unroll
  for (int j = 0; j < 16; j++) acc[j] = 0.0f;
  const int steps = kh / 8;
#pragma unroll 4
  for (int s = 0; s < steps; s++) {
    const u32x4_t wa = *reinterpret_cast<const u32x4_t *>(wp + 8 * s);
    const u32x4_t xb = load_x8<XT>(xp + 8 * s);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, wa), __builtin_bit_cast(bf16x8_t, xb),
                                                  acc, 0, 0, 0);
  }

  __shared__ float red[kWaves - 1][16][64];
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < 16; j++) red[wave - 1][j][lane] = acc[j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kWaves - 1; w++)
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] += red[w][j][lane];
  // accumulator j of this lane: row 8(j/4) + 4h + (j%4) of the tile, input c
  const int i = i0 + c;
  if (i >= a.n) return;
  float *const out = gridDim.z > 1 ? a.partial + (size_t)blockIdx.z * a.n * a.ldo : a.out;
  float *orow = out + (size_t)i * a.ldo + r0;
#pragma unroll
  for (int jq = 0; jq < 4; jq++) {
    const int rr = 8 * jq + 4 * h;
    if (a.ldo % 4 == 0 && r0 + rr + 3 < a.rows && (reinterpret_cast<uintptr_t>(orow + rr) & 15) == 0) {
      *reinterpret_cast<f32x4_t *>(orow + rr) = f32x4_t{acc[4 * jq], acc[4 * jq + 1], acc[4 * jq + 2], acc[4 * jq + 3]};
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (r0 + rr + e < a.rows) orow[rr + e] = acc[4 * jq + e];
    }
  }
}

// out[i][r] = sum over k of partial[k][i][r], k = 0 .. ksplit-1 in order.
__global__ __launch_bounds__(256) void matvec_sum_kernel(const MatvecArgs a) {
  const int r = (blockIdx.x * 256 + threadIdx.x) * 4;
  const int i = blockIdx.y;
  if (r >= a.rows) return;
  const size_t plane = (size_t)a.n * a.ldo;
  const float *p = a.partial + (size_t)i * a.ldo + r;
  float *o = a.out + (size_t)i * a.ldo + r;
  if (r + 3 < a.rows && a.ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(o) & 15) == 0) {
    f32x4_t acc = *reinterpret_cast<const f32x4_t *>(p);
    for (int k = 1; k < a.ksplit; k++) acc += *reinterpret_cast<const f32x4_t *>(p + k * plane);
    *reinterpret_cast<f32x4_t *>(o) = acc;
  } else {
    for (int e = 0; e < 4 && r + e < a.rows; e++) {
      float acc = p[e];
      for (int k = 1; k < a.ksplit; k++) acc += p[k * plane + e];
      o[e] = acc;
    }
  }
}

// The same sum with the slice count fixed at compile time: the KS loads of a
// lane are unrolled and all issued before the first add (the runtime-count loop
// above waits for each load in turn), and 64-lane workgroups spread the few
// rows over more compute units.  Same order of additions, same result.
template <int KS>
__global__ __launch_bounds__(64) void matvec_sum_fixed_kernel(const MatvecArgs a) {
  const int r = (blockIdx.x * 64 + threadIdx.x) * 4;
  const int i = blockIdx.y;
  if (r >= a.rows) return;
  const size_t plane = (size_t)a.n * a.ldo;
  const float *p = a.partial + (size_t)i * a.ldo + r;
  float *o = a.out + (size_t)i * a.ldo + r;
  f32x4_t v[KS];
#pragma unroll
  for (int k = 0; k < KS; k++) v[k] = *reinterpret_cast<const f32x4_t *>(p + k * plane);
  f32x4_t acc = v[0];
#pragma unroll
  for (int k = 1; k < KS; k++) acc += v[k];
  *reinterpret_cast<f32x4_t *>(o) = acc;
}

}  // namespace

int matvec_ksplit(int rows, int cols, int n, int cus) {
  const int tiles = ((rows + 31) / 32) * ((n + 31) / 32);
  int ks = 1;
  while (ks < 16 && tiles * ks * 2 <= cus && cols % (2 * ks * kMatvecColsMultiple) == 0) ks *= 2;
  return ks;
}

hipError_t launch_matvec_bf16(const MatvecArgs &a, hipStream_t s) {
  if (a.rows <= 0 || a.n <= 0) return hipSuccess;
  const int ks = a.ksplit > 1 && a.partial ? a.ksplit : 1;
  const dim3 grid((a.rows + 31) / 32, (a.n + 31) / 32, ks);
  if (a.x_f32)
    hipLaunchKernelGGL(matvec_bf16_kernel<float>, grid, dim3(64 * kWaves), 0, s, a);
  else
    hipLaunchKernelGGL(matvec_bf16_kernel<uint16_t>, grid, dim3(64 * kWaves), 0, s, a);
  if (ks == 1) return hipGetLastError();
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.rows % 4 == 0 && a.ldo % 4 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0 && (ks == 2 || ks == 4 || ks == 8 || ks == 16)) {
    const dim3 g((a.rows / 4 + 63) / 64, a.n);
    switch (ks) {
      case 2: hipLaunchKernelGGL(matvec_sum_fixed_kernel<2>, g, dim3(64), 0, s, a); break;
      case 4: hipLaunchKernelGGL(matvec_sum_fixed_kernel<4>, g, dim3(64), 0, s, a); break;
      case 8: hipLaunchKernelGGL(matvec_sum_fixed_kernel<8>, g, dim3(64), 0, s, a); break;
      default: hipLaunchKernelGGL(matvec_sum_fixed_kernel<16>, g, dim3(64), 0, s, a); break;
    }
  } else {
    hipLaunchKernelGGL(matvec_sum_kernel, dim3((a.rows + 1023) / 1024, a.n), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace llh
