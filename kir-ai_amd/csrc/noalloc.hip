// llh_paged_decode_noalloc: the paged decode step of llh_paged_decode with its
// split partials and merge descriptors in the library's own static device
// array instead of a stream workspace, so a call allocates nothing, ever.
// It is for callers that cannot call hipMalloc (code under HIP graph capture,
// tight serving loops, harnesses that forbid it); the reference has no
// counterpart (its Metal path allocates per command buffer).
//
// The array lives in this file's code object: every GPU the library runs on
// holds its own copy at its own address, for as long as the process lives.
// Host code never uses the array's name as an address (in host code it is a
// stand-in, not device memory): llh_ctx_create calls noalloc_init with its
// device current, which looks up that device's address once with
// hipGetSymbolAddress and keeps it, and the entry point passes that pointer to
// the kernels.  All calls on one GPU share the array, so calls that overlap on
// one GPU (on different streams or from different threads) race on it; the
// decode kernels write every partial and descriptor they read within the call,
// so nothing in it must start at zero.
#include <mutex>

#include "host_state.h"

namespace {

constexpr size_t kScratchBytes = LLH_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices] = {};  // device address of `scratch` per device

void *scratch_of(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_mu);
  return g_scratch[device];
}

}  // namespace

// Called by llh_ctx_create with `device` current: resolves this device's copy
// of the scratch array once.
int llh::noalloc_init(int device) {
  if (device < 0 || device >= kMaxDevices) return LLH_ERR_DEVICE;
  std::lock_guard<std::mutex> g(g_mu);
  if (g_scratch[device]) return LLH_OK;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) return LLH_ERR_DEVICE;
  g_scratch[device] = p;
  return LLH_OK;
}

extern "C" int llh_paged_decode_noalloc(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc,
                                        const void *d_q, void *d_out, float score_scale, void *stream) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  if (!d_out && desc->num_seqs > 0) return ctx->fail(LLH_ERR_NULL, "null device pointer in decode call");
  llh::DecodePlan plan;
  int st = llh::plan_decode(ctx, pool, desc, d_q, d_out, score_scale, &plan, kScratchBytes);
  if (st != LLH_OK || plan.empty) return st;
  if (plan.bytes > kScratchBytes)
    return ctx->fail(LLH_ERR_CAPACITY, "decode step needs " + std::to_string(plan.bytes) +
                                           " bytes of scratch; llh_paged_decode_noalloc holds " +
                                           std::to_string(kScratchBytes) + " (use llh_paged_decode)");
  char *base = static_cast<char *>(scratch_of(ctx->device));
  if (!base) return ctx->fail(LLH_ERR_DEVICE, "no-allocation scratch not resolved for this device");
  // flags go to the stream's own error word if it has one (finding it allocates
  // nothing), else to the context's
  int32_t *err = ctx->d_err;
  {
    std::lock_guard<std::mutex> g(ctx->ws_mu);
    for (auto &w : ctx->workspaces)
      if (w->stream == static_cast<hipStream_t>(stream) && w->err) err = w->err;
  }
  return llh::launch_planned_decode(ctx, pool, desc, plan, d_q, d_out, score_scale, static_cast<hipStream_t>(stream),
                                    base, err, /*timed=*/false);
}
