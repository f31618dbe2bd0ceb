"""The whole-block KV write kernel's shared-divisor quotient (div_shared in
kir-ai_amd/csrc/device_common.h, used by write_blocks_d128_kernel for int8 and fp8
pools) gives the codes of the correctly rounded division for every input it can see:
tests/quotient_check.c runs all of them (every bf16 absmax, the scale the kernel
derives from it, every bf16 element up to it) under IEEE and flush-to-zero
arithmetic.  The GPU tests hold the kernel's bytes to the oracle's quantisers on
sampled rows (tests/test_gpu_kv.py); this pins the arithmetic identity for all rows.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.fail("gcc is needed to build tests/quotient_check.c")
    exe = str(tmp_path_factory.mktemp("qc") / "quotient_check")
    flags = ["-O2", "-mfma", "-mf16c", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "quotient_check.c"), "-lm"]
    if subprocess.run([gcc, "-fopenmp"] + flags, capture_output=True).returncode != 0:
        subprocess.run([gcc] + flags, check=True)  # single-threaded without OpenMP
    return exe


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_shared_divisor_quotient_is_exact(checker, fmt):
    env = dict(os.environ, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "8"))
    r = subprocess.run([checker, fmt], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    fields = dict(kv.split("=") for kv in r.stdout.split()[1:])
    assert int(fields["pairs"]) > (1.7e8 if fmt == "int8" else 1.0e9)
    assert fields["mismatches_ieee"] == "0" and fields["mismatches_ftz"] == "0"
