"""Shared pytest setup.

Tests marked ``gpu`` call the HIP library through its C ABI on cuda:0; they
fail (not skip) when no GPU is visible, so a silent host fallback cannot pass.
Everything else runs on the CPU: the oracle against the reference's golden
vectors, host logic, and that the C-ABI library loads and exports its symbols.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "kir-ai_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def ctx():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import llm_hip

    c = llm_hip.Context(0)
    yield c
    c.close()


@pytest.fixture
def opts(ctx):
    """set(option, value) for one test: context tuning options (llh_ctx_set_option),
    restored to their previous values afterwards."""
    import llm_hip

    saved = {}

    def set_(option, value):
        if option not in saved:
            saved[option] = ctx.get_option(option)
        if option == llm_hip.OPT_DECODE_KERNEL and isinstance(value, str):
            value = llm_hip.DECODE_KERNELS[value]
        ctx.set_option(option, value)

    yield set_
    for o, v in saved.items():
        ctx.set_option(o, v)
