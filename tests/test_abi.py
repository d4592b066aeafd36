"""The C-ABI library (include/moe_mi355x.h) on the CPU: it loads into a torch
process, exports every declared entry point, the Python binding covers exactly
that set, host-side argument validation returns the documented status codes
without launching anything, and the product path refuses to run off the GPU."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_mi355x.h")


def declared_symbols() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"^(?:int|int64_t)\s+(moe_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    from torchtitan_amd import _lib

    if not os.path.exists(_lib.library_path()):
        from torchtitan_amd import build

        build.build()
    return _lib.lib()


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 18
    assert {"moe_router_fwd", "moe_reorder", "moe_permute", "moe_combine", "moe_grouped_gemm_gate_up"} <= syms


def test_library_exports_every_declared_symbol(lib):
    from torchtitan_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", _lib.library_path()], capture_output=True, text=True)
    exported = set(re.findall(r"\bT\s+(moe_\w+)", out.stdout))
    missing = declared_symbols() - exported
    assert not missing, f"declared but not exported: {missing}"
    for name in declared_symbols():
        assert getattr(lib, name) is not None


def test_binding_covers_the_header(lib):
    from torchtitan_amd import _lib

    assert set(_lib.SIGNATURES) == declared_symbols()


def test_host_side_validation_returns_status_codes(lib):
    """Invalid shapes are rejected before any launch (no GPU needed)."""
    null = None
    # router: zero experts, top_k > experts, bad score function
    assert lib.moe_router_fwd(null, null, 4, 0, 1, 1, 0, 0, 0, 1.0, 0, null, null, null, null) == -1
    assert lib.moe_router_fwd(null, null, 4, 4, 5, 1, 0, 0, 0, 1.0, 0, null, null, null, null) == -1
    assert lib.moe_router_fwd(null, null, 4, 8, 2, 7, 0, 0, 0, 1.0, 0, null, null, null, null) == -1
    # group limit: E not divisible by groups, one expert per group
    assert lib.moe_router_fwd(null, null, 4, 10, 2, 1, 3, 1, 0, 1.0, 0, null, null, null, null) == -1
    assert lib.moe_router_fwd(null, null, 4, 8, 2, 1, 8, 2, 0, 1.0, 0, null, null, null, null) == -1
    # zero tokens is a no-op
    assert lib.moe_router_fwd(null, null, 0, 8, 2, 1, 0, 0, 0, 1.0, 0, null, null, null, null) == 0
    # workspace size and a too-small workspace
    assert lib.moe_reorder_workspace_bytes(1000, 256) == 2 * 4 * 256 * 4
    assert lib.moe_reorder(null, null, 1000, 8, 256, null, 16, null, null, null, null, null, null, null) == -4
    # rows: dims that are not whole 16-byte chunks
    assert lib.moe_permute(null, null, null, 4, 12, 2, 0, null, null) == -1
    assert lib.moe_combine(null, null, null, null, 4, 6, 2, 1, null, null) == -1
    # grouped GEMM shape rules: dims below 64 are invalid, dims not a multiple of 64 unsupported
    assert lib.moe_grouped_gemm_gate_up(null, null, null, null, 8, 4, 32, 256, null, null, null, null) == -1
    assert lib.moe_grouped_gemm_gate_up(null, null, null, null, 8, 4, 768 + 32, 256, null, null, null, null) == -2
    assert lib.moe_grouped_gemm_oss_gate_up(null, null, null, null, 8, 4, 2880, 2880 + 16, 7.0, null, null, null,
                                            null) == -2
    # the fp8 / MXFP8 kernels keep D, H multiples of 256
    assert lib.moe_fp8_gemm_down(null, null, null, null, null, 8, 4, 768 + 64, 256, null, null) == -2
    assert lib.moe_mxfp8_gemm_down(null, null, null, null, null, 8, 4, 768 + 64, 256, null, null) == -2
    assert lib.moe_grouped_gemm_bwd_dw2(null, null, null, 8, 0, 256, 256, null, null) == -1
    # the SwiGLU epilogues' pointwise test entry: a negative count or missing buffers
    # are refused, an empty one is a no-op
    assert lib.moe_swiglu_pointwise_f32(null, null, null, -1, null) == -1
    assert lib.moe_swiglu_pointwise_f32(null, null, null, 4, null) == -1
    assert lib.moe_swiglu_pointwise_f32(null, null, null, 0, null) == 0


def test_status_codes_map_to_exceptions():
    from torchtitan_amd import _lib

    with pytest.raises(_lib.MoEKernelError, match="workspace too small"):
        _lib.check(-4, "moe_reorder")
    _lib.check(0, "ok")


def test_ops_refuse_cpu_tensors():
    """No CPU or eager fallback: the product path raises off the GPU."""
    from torchtitan_amd import _lib, ops

    with pytest.raises(_lib.MoEKernelError, match="GPU"):
        ops.router(torch.zeros(4, 8), None, 8, 2, 1, 0, 0, False, 1.0, False)
    with pytest.raises(_lib.MoEKernelError, match="GPU"):
        ops.grouped_swiglu(torch.zeros(4, 256, dtype=torch.bfloat16), torch.zeros(1, 256, 256, dtype=torch.bfloat16),
                           torch.zeros(1, 256, 256, dtype=torch.bfloat16), torch.zeros(1, 256, 256, dtype=torch.bfloat16),
                           torch.tensor([4]))


def test_missing_library_raises(monkeypatch, tmp_path):
    from torchtitan_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "_LIB_PATH", str(tmp_path / "libmoe_mi355x.so"))
    with pytest.raises(_lib.MoEKernelError, match="missing"):
        _lib.lib()
