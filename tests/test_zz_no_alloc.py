"""moe_reorder_noalloc, the reorder entry point that allocates nothing (its
workspace is a fixed device array of MOE_REORDER_NOALLOC_SCRATCH_BYTES), called
through the C ABI against moe_reorder on the same inputs: every output
bit-identical, on two calls in a row with the second smaller (the scratch keeps
the first call's contents), then a request past the array's size is refused
with MOE_ERR_WORKSPACE before anything is launched."""

import ctypes

import pytest
import torch

from tests.conftest import banner

pytestmark = pytest.mark.gpu

MOE_ERR_WORKSPACE = -4
SCRATCH_BYTES = 4 << 20


def _routing(n, e, k, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    scores = torch.rand(n, e, generator=g, device=dev)
    idx = torch.topk(scores, k, dim=1, sorted=False).indices.contiguous()
    top = torch.rand(n, k, generator=g, device=dev)
    return idx, top


def _outputs(n, e, k, dev):
    r = n * k
    return {
        "scores_sorted": torch.full((r,), -1.0, device=dev),
        "token_idx": torch.full((r,), -1, dtype=torch.int64, device=dev),
        "counts": torch.full((e,), -1, dtype=torch.int64, device=dev),
        "offsets": torch.full((e,), -1, dtype=torch.int32, device=dev),
        "slot_pos": torch.full((n, k), -1, dtype=torch.int32, device=dev),
        "tok_pos": torch.full((n, k), -1, dtype=torch.int32, device=dev),
    }


def _ptrs(o):
    return [o[k].data_ptr() for k in ("scores_sorted", "token_idx", "counts", "offsets", "slot_pos", "tok_pos")]


def test_reorder_noalloc_matches_reorder(dev):
    from torchtitan_amd import _lib

    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    for n, e, k, seed in ((32768, 256, 8, 1), (1000, 64, 6, 2)):  # the second call is smaller
        banner(f"reorder_noalloc vs reorder: n={n} e={e} k={k}")
        idx, top = _routing(n, e, k, dev, seed)
        ref, got = _outputs(n, e, k, dev), _outputs(n, e, k, dev)
        nbytes = lib.moe_reorder_workspace_bytes(n, e)
        assert nbytes <= SCRATCH_BYTES
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.moe_reorder(idx.data_ptr(), top.data_ptr(), n, k, e, ws.data_ptr(), nbytes, *_ptrs(ref),
                                   stream), "moe_reorder")
        _lib.check(lib.moe_reorder_noalloc(idx.data_ptr(), top.data_ptr(), n, k, e, *_ptrs(got), stream),
                   "moe_reorder_noalloc")
        torch.cuda.synchronize()
        for name in ref:
            assert torch.equal(got[name], ref[name]), name
        assert int(got["counts"].sum()) == n * k


def test_reorder_noalloc_rejects_sizes_past_its_scratch(dev):
    from torchtitan_amd import _lib

    lib = _lib.lib()
    n, e, k = 600000, 256, 8  # 2 * ceil(n / 256) * 256 * 4 bytes > 4 MiB
    assert lib.moe_reorder_workspace_bytes(n, e) > SCRATCH_BYTES
    # null pointers: whichever check ran first, the call returns an error and
    # launches nothing
    p = ctypes.c_void_p(None)
    st = lib.moe_reorder_noalloc(p, p, n, k, e, p, p, p, p, p, p, torch.cuda.current_stream(dev).cuda_stream)
    assert st == MOE_ERR_WORKSPACE
