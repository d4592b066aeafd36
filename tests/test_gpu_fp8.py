"""fp8 e4m3 grouped SwiGLU experts on the GPU.

Parity is unpinned against the reference (its fp8 path is torchao's, absent
here); the kernels are checked against the oracle's restatement of that
recipe (experts_fp8_forward / experts_fp8_backward) and, with a looser bound,
against the bf16 experts:
  * quantizers: fp8 bytes and scales bit-exact vs the oracle;
  * each fp8 GEMM entry point, fed the oracle's own quantized operands:
    normwise relative error <= 1e-2 (only the fp32 summation order differs,
    so outputs differ by at most one bf16 rounding);
  * the chained op (fwd + bwd): <= 5e-2 vs the fp8 emulation, where a one-ulp
    bf16 difference can move a requantized fp8 value by one fp8 step, and
    <= 0.1 vs the fp32 reference on the bf16 inputs (fp8 quantization error).
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import moe_ref as R
from tests.conftest import banner

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-2
EMU_TOL = 5e-2
BF16_TOL = 0.1


def _rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def _u8(q):
    return q.view(torch.uint8).contiguous()


# experts, D, H, rows per expert: ragged with empty experts; tall experts over several
# 256-row m-tiles with partial last tiles; single-row and tile-edge groups
GEMM_SHAPES = {
    "ragged_e6_d256_h256": (6, 256, 256, [40, 0, 130, 17, 64, 3]),
    "tall_e3_d512_h768": (3, 512, 768, [700, 0, 517]),
    "edges_e5_d768_h256": (5, 768, 256, [1, 255, 257, 0, 390]),
}


@pytest.mark.parametrize("shape", list(GEMM_SHAPES))
def test_fp8_gemm_entry_points_match_emulation(dev, shape):
    """Every fp8 GEMM kernel against R._fp8_mm on identical quantized operands."""
    banner("fp8 GEMM entry points")
    from torchtitan_amd import _lib, ops

    e, d, h, counts = GEMM_SHAPES[shape]
    gen = torch.Generator().manual_seed(2)
    r = sum(counts)
    cnt = torch.tensor(counts, dtype=torch.int64)
    x = torch.randn(r, d, generator=gen).bfloat16()
    w1, w3 = ((torch.randn(e, h, d, generator=gen) * 0.05).bfloat16() for _ in range(2))
    w2 = (torch.randn(e, d, h, generator=gen) * 0.05).bfloat16()
    dy = torch.randn(r, d, generator=gen).bfloat16()
    gg = torch.randn(r, h, generator=gen).bfloat16()
    uu = torch.randn(r, h, generator=gen).bfloat16()
    dgu = torch.randn(r, 2 * h, generator=gen).bfloat16()
    hh = torch.randn(r, h, generator=gen).bfloat16()
    st = torch.cuda.current_stream().cuda_stream
    keep = []  # device copies must outlive the launches that read them

    def P(t):
        dt = t.to(dev).contiguous()
        keep.append(dt)
        return dt.data_ptr()
    cd = cnt.to(dev)
    segs = [(sum(counts[:i]), c) for i, c in enumerate(counts)]

    def per_expert(fn):
        return torch.cat([fn(i, slice(s0, s0 + c)) for i, (s0, c) in enumerate(segs)])

    # gate_up
    qx, sx = R.quant_fp8_rows(x)
    qw1, sw1 = R.quant_fp8_rows(w1)
    qw3, sw3 = R.quant_fp8_rows(w3)
    g_, u_, h_ = (torch.empty(r, h, dtype=torch.bfloat16, device=dev) for _ in range(3))
    _lib.call("moe_fp8_gemm_gate_up", P(_u8(qx)), P(sx), P(_u8(qw1)), P(sw1), P(_u8(qw3)), P(sw3), cd.data_ptr(),
              r, e, d, h, g_.data_ptr(), u_.data_ptr(), h_.data_ptr(), st)
    eg = per_expert(lambda i, sl: R._fp8_mm(qx[sl], sx[sl], qw1[i], sw1[i]).bfloat16())
    eu = per_expert(lambda i, sl: R._fp8_mm(qx[sl], sx[sl], qw3[i], sw3[i]).bfloat16())
    assert _rel(g_, eg) <= GEMM_TOL and _rel(u_, eu) <= GEMM_TOL
    # the epilogue's h from its own g and u is torch's silu(g) * u bit for bit
    assert torch.equal(h_, F.silu(g_) * u_)
    # down
    qh, sh = R.quant_fp8_rows(hh)
    qw2, sw2 = R.quant_fp8_rows(w2)
    y_ = torch.empty(r, d, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_fp8_gemm_down", P(_u8(qh)), P(sh), P(_u8(qw2)), P(sw2), cd.data_ptr(), r, e, d, h,
              y_.data_ptr(), st)
    assert _rel(y_, per_expert(lambda i, sl: R._fp8_mm(qh[sl], sh[sl], qw2[i], sw2[i]).bfloat16())) <= GEMM_TOL
    # bwd dgu (check dh through du = dh * bf16(silu(g)))
    qdy, sdy = R.quant_fp8_rows(dy)
    qw2t, sw2t = zip(*(R.quant_fp8_rows(w2[i].t()) for i in range(e)))
    qw2t, sw2t = torch.stack(qw2t), torch.stack(sw2t)
    dgu_ = torch.empty(r, 2 * h, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_fp8_gemm_bwd_dgu", P(_u8(qdy)), P(sdy), P(_u8(qw2t)), P(sw2t), P(gg), P(uu), cd.data_ptr(), r, e,
              d, h, dgu_.data_ptr(), st)
    dh = per_expert(lambda i, sl: R._fp8_mm(qdy[sl], sdy[sl], qw2t[i], sw2t[i]).bfloat16())
    assert _rel(dgu_[:, h:], dh * F.silu(gg)) <= GEMM_TOL
    assert _rel(dgu_[:, :h], torch.ops.aten.silu_backward(dh * uu, gg)) <= GEMM_TOL
    # bwd dx
    qdgu, sdgu = R.quant_fp8_rows(dgu.view(r, 2, h))
    qw1t, sw1t = zip(*(R.quant_fp8_rows(w1[i].t()) for i in range(e)))
    qw3t, sw3t = zip(*(R.quant_fp8_rows(w3[i].t()) for i in range(e)))
    qw13t = torch.cat([torch.stack(qw1t).view(torch.uint8), torch.stack(qw3t).view(torch.uint8)], dim=2)
    sw13t = torch.stack([torch.stack(sw1t).view(e, d), torch.stack(sw3t).view(e, d)], dim=1)
    dx_ = torch.empty(r, d, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_fp8_gemm_bwd_dx", P(_u8(qdgu)), P(sdgu), P(qw13t), P(sw13t), cd.data_ptr(), r, e, d, h,
              dx_.data_ptr(), st)
    qdg, sdg, qdu, sdu = qdgu[:, 0], sdgu[:, 0], qdgu[:, 1], sdgu[:, 1]
    edx = per_expert(lambda i, sl: R._fp8_mm(qdg[sl], sdg[sl], qw1t[i], sw1t[i]).bfloat16()
                     + R._fp8_mm(qdu[sl], sdu[sl], qw3t[i], sw3t[i]).bfloat16())
    assert _rel(dx_, edx) <= GEMM_TOL
    # bwd dw13 / dw2 from token-transposed, 16-padded operands
    rpad = ops._padded_rows(r, e)

    def tokens_t(t):
        c = t.shape[1]
        q = torch.zeros(c, rpad, dtype=torch.uint8)
        sc = torch.ones(e, c)
        qs, pstart = [], 0
        for i, (s0, n) in enumerate(segs):
            if n:
                qq, ss = R.quant_fp8_rows(t[s0:s0 + n].t())
                q[:, pstart:pstart + n] = qq.view(torch.uint8)
                sc[i] = ss.view(-1)
                qs.append((qq, ss))
            else:
                qs.append(None)
            pstart += (n + 127) // 128 * 128
        return q, sc, qs

    qdgut, sdgut, ldgu = tokens_t(dgu)
    qxt, sxt, lx = tokens_t(x)
    dw1_, dw3_ = torch.empty_like(w1, device=dev), torch.empty_like(w3, device=dev)
    _lib.call("moe_fp8_gemm_bwd_dw13", P(qdgut), P(sdgut), P(qxt), P(sxt), cd.data_ptr(), r, rpad, e, d, h,
              dw1_.data_ptr(), dw3_.data_ptr(), st)
    qdyt, sdyt, ldy = tokens_t(dy)
    qht, sht, lh = tokens_t(hh)
    dw2_ = torch.empty_like(w2, device=dev)
    _lib.call("moe_fp8_gemm_bwd_dw2", P(qdyt), P(sdyt), P(qht), P(sht), cd.data_ptr(), r, rpad, e, d, h,
              dw2_.data_ptr(), st)
    for i, (s0, n) in enumerate(segs):
        if n == 0:
            for t in (dw1_, dw2_, dw3_):
                assert torch.count_nonzero(t[i]) == 0
            continue
        (qa, sa), (qb, sb) = ldgu[i], lx[i]
        edw = R._fp8_mm(qa, sa, qb, sb).bfloat16()  # [2H, D]
        assert _rel(dw1_[i], edw[:h]) <= GEMM_TOL and _rel(dw3_[i], edw[h:]) <= GEMM_TOL
        (qa, sa), (qb, sb) = ldy[i], lh[i]
        assert _rel(dw2_[i], R._fp8_mm(qa, sa, qb, sb).bfloat16()) <= GEMM_TOL


def test_fp8_quantizers_bit_exact(dev):
    banner("fp8 quantizers")
    from torchtitan_amd import _lib, ops

    g = torch.Generator().manual_seed(0)
    x = (torch.randn(300, 512, generator=g) * torch.exp(torch.randn(300, 1, generator=g) * 3)).bfloat16()
    x[7] = 0  # all-zero row
    q, s = ops._quant_rows(x.to(dev), 512)
    rq, rs = R.quant_fp8_rows(x)
    assert torch.equal(q.cpu(), rq.view(torch.uint8)), "row-quantized bytes differ"
    assert torch.equal(s.cpu(), rs.view(-1))
    # columns, transposed: w [E, A, B] -> [E, B, A]
    e, a, b = 3, 256, 128
    w = torch.randn(e, a, b, generator=g).bfloat16()
    qt = torch.empty(e, b, a, dtype=torch.uint8, device=dev)
    st = torch.empty(e, b, dtype=torch.float32, device=dev)
    wd = w.to(dev)
    _lib.call("moe_fp8_quant_cols_t", wd.data_ptr(), e, a, b, qt.data_ptr(), b * a, a, st.data_ptr(), b,
              torch.cuda.current_stream().cuda_stream)
    for i in range(e):
        rq, rs = R.quant_fp8_rows(w[i].t())
        assert torch.equal(qt[i].cpu(), rq.view(torch.uint8))
        assert torch.equal(st[i].cpu(), rs.view(-1))
    # token groups, transposed and 16-padded
    counts = torch.tensor([5, 0, 33, 16, 1], dtype=torch.int64)
    r, c = int(counts.sum()), 128
    xt = torch.randn(r, c, generator=g).bfloat16()
    rpad = ops._padded_rows(r, len(counts))
    q2, s2 = ops._quant_tokens_t(xt.to(dev), counts.to(dev), len(counts), rpad)
    q2, s2 = q2.cpu(), s2.cpu()
    start = pstart = 0
    for i, n in enumerate(counts.tolist()):
        if n:
            rq, rs = R.quant_fp8_rows(xt[start:start + n].t())
            assert torch.equal(q2[:, pstart:pstart + n], rq.view(torch.uint8))
            pad = (n + 127) // 128 * 128
            assert torch.count_nonzero(q2[:, pstart + n:pstart + pad]) == 0
            assert torch.equal(s2[i], rs.view(-1))
        start += n
        pstart += (n + 127) // 128 * 128



@pytest.mark.parametrize("shape", [(8, 1024, 2304), (4, 2304, 1024), (3, 100, 264), (2, 37, 4096)])
def test_fp8_weight_quantizers_from_two_reads(dev, shape):
    """moe_fp8_quant_rows_colamax: the row-quantized bytes and scales equal the
    oracle's (as moe_fp8_quant_rows), and the column amax equals max |x| over the
    rows; moe_fp8_quant_cols_t_amax from that amax equals the oracle's transposed
    quantization. With an inf and NaNs planted (which the oracle's unsaturated cast
    and NaN-propagating amax do not model), the two-read path still equals the
    kernels that find their own amax: moe_fp8_quant_rows and moe_fp8_quant_cols_t
    (NaN ignored by the amax, as fmaxf does)."""
    from torchtitan_amd import _lib, ops

    e, a, b = shape
    banner(f"fp8 weight quantizers {shape}")
    g = torch.Generator().manual_seed(a + b)
    w = (torch.randn(e, a, b, generator=g) * torch.exp(torch.randn(e, a, 1, generator=g) * 2)).bfloat16()
    w[0, 3] = 0  # an all-zero row
    stream = torch.cuda.current_stream().cuda_stream
    transposable = a % 16 == 0 and b % 64 == 0  # the transposing quantizers' shape rule

    def two_read(wd):
        q, sc, amax = ops._quant_rows_colamax(wd)
        qt = st = None
        if transposable:
            qt = torch.empty(e, b, a, dtype=torch.uint8, device=dev)
            st = torch.empty(e, b, dtype=torch.float32, device=dev)
            ops._quant_cols_t(wd, amax, qt, 0, b * a, a, st, 0, b)
        return q, sc, amax, qt, st

    q, sc, amax, qt, st = two_read(w.to(dev))
    rq, rs = R.quant_fp8_rows(w.view(e * a, b))
    assert torch.equal(q.view(e * a, b).cpu(), rq.view(torch.uint8))
    assert torch.equal(sc.cpu(), rs.view(-1))
    assert torch.equal(amax.cpu(), w.float().abs().amax(dim=1))
    if transposable:
        for i in range(e):
            rq, rs = R.quant_fp8_rows(w[i].t())
            assert torch.equal(qt[i].cpu(), rq.view(torch.uint8))
            assert torch.equal(st[i].cpu(), rs.view(-1))
    # non-finite values: against the one-read-per-layout kernels
    w[e - 1, a // 2, 5] = float("inf")
    w[0, 1, 7] = float("nan")
    w[e - 1, :, 9] = float("nan")  # a column of NaN: amax 0
    wd = w.to(dev)
    q, sc, amax, qt, st = two_read(wd)
    q1, s1 = ops._quant_rows(wd, b)
    assert torch.equal(q.view(e * a, b), q1.view(e * a, b)) and torch.equal(sc, s1)
    wf = w.float().abs()
    assert torch.equal(amax.cpu(), torch.where(torch.isnan(wf), torch.zeros_like(wf), wf).amax(dim=1))
    if transposable:
        qt2, st2 = torch.empty_like(qt), torch.empty_like(st)
        _lib.call("moe_fp8_quant_cols_t", wd.data_ptr(), e, a, b, qt2.data_ptr(), b * a, a, st2.data_ptr(), b, stream)
        assert torch.equal(qt, qt2) and torch.equal(st, st2)


TOKEN_CASES = {
    # (rows, cols, pieces, counts): rows past the last group, an empty group, a
    # piece boundary inside a lane's chunk run (640 columns), 64-column slabs
    # (192), the widest rows (8192)
    "d2304_tail": (700, 2304, 1, [100, 0, 333, 7, 200]),
    "dgu_2x640": (513, 1280, 2, [256, 1, 256]),
    "d192": (300, 192, 1, [17, 0, 0, 283]),
    "d8192": (300, 8192, 1, [50, 150, 0, 100]),
}


@pytest.mark.parametrize("name", list(TOKEN_CASES))
def test_fp8_token_quantizers_from_two_reads(dev, name):
    """moe_fp8_quant_rows_groupamax: the row-quantized bytes and the scale of each
    row piece equal the oracle's (as moe_fp8_quant_rows over cols / pieces), and
    the amax of each (group, column) equals max |x| over the group's rows (rows
    past the last group enter none); moe_fp8_quant_tokens_t_amax from that amax
    equals the oracle's per-group transposed quantization. With an inf and NaNs
    planted, both still equal the kernels that find their own amax (NaN ignored
    by the amax, as fmaxf does)."""
    from torchtitan_amd import ops

    r, c, pieces, counts = TOKEN_CASES[name]
    banner(f"fp8 token quantizers {name}")
    g = torch.Generator().manual_seed(r + c)
    x = (torch.randn(r, c, generator=g) * torch.exp(torch.randn(r, 1, generator=g) * 2)).bfloat16()
    x[3] = 0  # an all-zero row
    e = len(counts)
    cnt = torch.tensor(counts, dtype=torch.int64)
    cd = cnt.to(dev)
    rpad = ops._padded_rows(r, e)

    def absmax(t):
        t = t.float().abs()
        return torch.where(torch.isnan(t), torch.zeros_like(t), t).amax(dim=0)

    def check_amax(amax):
        start = 0
        for i, n in enumerate(counts):
            want = absmax(x[start:start + n]) if n else torch.zeros(c)
            assert torch.equal(amax[i].cpu(), want), f"group {i}"
            start += n

    xd = x.to(dev)
    q, sc, amax = ops._quant_rows_groupamax(xd, cd, e, pieces)
    rq, rs = R.quant_fp8_rows(x.view(r * pieces, c // pieces))
    assert torch.equal(q.cpu().view(r * pieces, c // pieces), rq.view(torch.uint8))
    assert torch.equal(sc.cpu(), rs.view(-1))
    check_amax(amax)
    qt, st = ops._quant_tokens_t(xd, cd, e, rpad, amax)
    qt, st = qt.cpu(), st.cpu()
    start = pstart = 0
    for i, n in enumerate(counts):
        if n:
            rq, rs = R.quant_fp8_rows(x[start:start + n].t())
            assert torch.equal(qt[:, pstart:pstart + n], rq.view(torch.uint8)), f"group {i}"
            assert torch.count_nonzero(qt[:, pstart + n:pstart + (n + 127) // 128 * 128]) == 0
            assert torch.equal(st[i], rs.view(-1))
        start += n
        pstart += (n + 127) // 128 * 128
    # non-finite values: against the kernels that take their own amax
    x[5, 7] = float("inf")
    x[1, 2] = float("nan")
    x[:, 9] = float("nan")  # a column of NaN: amax 0
    xd = x.to(dev)
    q, sc, amax = ops._quant_rows_groupamax(xd, cd, e, pieces)
    q1, s1 = ops._quant_rows(xd, c // pieces)
    assert torch.equal(q.view(-1), q1.view(-1)) and torch.equal(sc, s1)
    check_amax(amax)
    qt, st = ops._quant_tokens_t(xd, cd, e, rpad, amax)
    qt1, st1 = ops._quant_tokens_t(xd, cd, e, rpad)
    assert torch.equal(qt[:, :pstart], qt1[:, :pstart])
    full = cnt > 0  # empty groups write no scale
    assert torch.equal(st[full.to(dev)], st1[full.to(dev)])


@pytest.mark.parametrize("width", [192, 320, 384])
def test_fp8_transposing_quantizers_slab_widths(dev, width):
    """The transposing quantizers at widths that take 64-column slabs (192, 320)
    and 128-column ones (384): bit-exact against the oracle as at width 128."""
    banner(f"fp8 transposing quantizers width={width}")
    g = torch.Generator().manual_seed(width)
    from torchtitan_amd import _lib, ops
    e, a = 3, 256
    w = torch.randn(e, a, width, generator=g).bfloat16()
    qt = torch.empty(e, width, a, dtype=torch.uint8, device=dev)
    st = torch.empty(e, width, dtype=torch.float32, device=dev)
    _lib.call("moe_fp8_quant_cols_t", w.to(dev).data_ptr(), e, a, width, qt.data_ptr(), width * a, a, st.data_ptr(),
              width, torch.cuda.current_stream().cuda_stream)
    for i in range(e):
        rq, rs = R.quant_fp8_rows(w[i].t())
        assert torch.equal(qt[i].cpu(), rq.view(torch.uint8))
        assert torch.equal(st[i].cpu(), rs.view(-1))
    counts = torch.tensor([5, 0, 300, 16, 1], dtype=torch.int64)
    r = int(counts.sum())
    xt = torch.randn(r, width, generator=g).bfloat16()
    rpad = ops._padded_rows(r, len(counts))
    q2, s2 = ops._quant_tokens_t(xt.to(dev), counts.to(dev), len(counts), rpad)
    q2, s2 = q2.cpu(), s2.cpu()
    start = pstart = 0
    for i, n in enumerate(counts.tolist()):
        if n:
            rq, rs = R.quant_fp8_rows(xt[start:start + n].t())
            assert torch.equal(q2[:, pstart:pstart + n], rq.view(torch.uint8))
            assert torch.equal(s2[i], rs.view(-1))
        start += n
        pstart += (n + 127) // 128 * 128

CASES = {
    "ragged_e8": (8, 256, 512, [37, 0, 130, 16, 255, 1, 64, 100]),
    "e16_d512_h256": (16, 512, 256, [96, 81, 0, 0, 200, 17, 33, 64, 128, 5, 70, 90, 300, 2, 0, 40]),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fp8_grouped_swiglu_fwd_bwd(dev, name):
    e, d, h, counts = CASES[name]
    banner(f"fp8 grouped swiglu {name}")
    from torchtitan_amd import ops

    g = torch.Generator().manual_seed(1)
    r = sum(counts)
    x = torch.randn(r, d, generator=g).bfloat16()
    w1 = (torch.randn(e, h, d, generator=g) * 0.05).bfloat16()
    w2 = (torch.randn(e, d, h, generator=g) * 0.05).bfloat16()
    w3 = (torch.randn(e, h, d, generator=g) * 0.05).bfloat16()
    dy = torch.randn(r, d, generator=g).bfloat16()
    cnt = torch.tensor(counts, dtype=torch.int64)
    xs, a, b, c = (t.to(dev).requires_grad_(True) for t in (x, w1, w2, w3))
    y, gg, uu, hh, *_ = ops.grouped_swiglu_fp8(xs, a, b, c, cnt.to(dev))
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    # fp8 emulation
    ey, eg, eu, eh = R.experts_fp8_forward(w1, w2, w3, x, cnt)
    edx, edw1, edw2, edw3 = R.experts_fp8_backward(w1, w2, w3, x, cnt, eg, eu, eh, dy)
    errs = {"y": _rel(y, ey), "g": _rel(gg, eg), "h": _rel(hh, eh), "dx": _rel(xs.grad, edx),
            "dw1": _rel(a.grad, edw1), "dw2": _rel(b.grad, edw2), "dw3": _rel(c.grad, edw3)}
    print(f"[case] {name} vs fp8 emulation: {errs}", flush=True)
    assert all(v <= EMU_TOL for v in errs.values()), errs
    for i, n in enumerate(counts):
        if n == 0:
            for t in (a.grad, b.grad, c.grad):
                assert torch.count_nonzero(t[i]) == 0
    # against the fp32 reference on the same bf16 inputs
    xr, w1r, w2r, w3r = (t.float().requires_grad_(True) for t in (x, w1, w2, w3))
    ys, start = [], 0
    for i, n in enumerate(counts):
        xe = xr[start:start + n]
        ys.append((F.silu(xe @ w1r[i].t()) * (xe @ w3r[i].t())) @ w2r[i].t())
        start += n
    yr = torch.cat(ys)
    yr.backward(dy.float())
    loose = {"y": _rel(y, yr), "dx": _rel(xs.grad, xr.grad), "dw1": _rel(a.grad, w1r.grad),
             "dw2": _rel(b.grad, w2r.grad), "dw3": _rel(c.grad, w3r.grad)}
    print(f"[case] {name} vs fp32 reference: {loose}", flush=True)
    assert all(v <= BF16_TOL for v in loose.values()), loose


def test_fp8_quantizers_nan_elements(dev):
    """A NaN element quantizes to 0x7f and sends only its own wave (row-wise) or
    LDS tile (transposed) to the software conversion: every row and column
    without a NaN still matches the oracle bit for bit. (The NaN row's or
    column's scale is not compared: the kernels' amax skips NaN, torch's
    propagates it.)"""
    banner("fp8 quantizers with NaN elements")
    from torchtitan_amd import ops

    g = torch.Generator().manual_seed(5)
    x = torch.randn(256, 512, generator=g).bfloat16()
    x[13, 5] = float("nan")
    q, _ = ops._quant_rows(x.to(dev), 512)
    q = q.cpu()
    rq, _ = R.quant_fp8_rows(x)
    keep = torch.ones(256, dtype=torch.bool)
    keep[13] = False
    assert q[13, 5].item() == 0x7F
    assert torch.equal(q[keep], rq.view(torch.uint8)[keep])
    # token groups, transposed: the NaN's tile takes the software path
    counts = torch.tensor([100, 0, 156], dtype=torch.int64)
    xt = torch.randn(256, 128, generator=g).bfloat16()
    xt[40, 70] = float("nan")
    rpad = ops._padded_rows(256, 3)
    q2, _ = ops._quant_tokens_t(xt.to(dev), counts.to(dev), 3, rpad)
    q2 = q2.cpu()
    assert q2[70, 40].item() == 0x7F
    cols = torch.ones(128, dtype=torch.bool)
    cols[70] = False
    rq0, _ = R.quant_fp8_rows(xt[0:100].t())
    rq2, _ = R.quant_fp8_rows(xt[100:256].t())
    assert torch.equal(q2[cols, 0:100], rq0.view(torch.uint8)[cols])
    assert torch.equal(q2[:, 128:284], rq2.view(torch.uint8))  # group 2 at ceil128(100)


@pytest.mark.parametrize("cols", [2304, 192])
@pytest.mark.parametrize("scaled", [True, False])
def test_fp8_gathering_token_quantizers_match_permute_then_quantize(dev, cols, scaled):
    """moe_fp8_quant_rows_groupamax_gather and moe_fp8_quant_tokens_t_amax_gather
    read the routed rows x[token_idx] (* score, rounded to bf16) in place: bytes,
    scales and group amax identical to the permute op's output fed to the
    non-gathering quantizers (ragged groups, an empty expert, 64-column slabs)."""
    banner(f"fp8 gathering token quantizers cols={cols} scaled={scaled}")
    from torchtitan_amd import ops

    g = torch.Generator().manual_seed(12)
    n, e, k = 300, 8, 2
    x = (torch.randn(n, cols, generator=g) * 3).bfloat16().to(dev)
    logits = torch.randn(n, e, generator=g)
    logits[:, 5] = -1e9  # expert 5 receives no token
    top, idx = logits.topk(k, dim=1)
    scores_sorted, token_idx, counts, _offs, slot_pos, tok_pos = ops.reorder(top.sigmoid().to(dev), idx.to(dev), e)
    sc = scores_sorted if scaled else None
    routed = ops.permute(x, slot_pos, tok_pos, sc)
    q1, s1, a1 = ops._quant_rows_groupamax(routed, counts, e)
    q2, s2, a2 = ops._quant_rows_groupamax_gather(x, token_idx, sc, counts, e)
    assert torch.equal(q1, q2) and torch.equal(s1, s2) and torch.equal(a1, a2)
    rpad = ops._padded_rows(n * k, e)
    qt1, st1 = ops._quant_tokens_t(routed, counts, e, rpad, a1)
    qt2, st2 = ops._quant_tokens_t_gather(x, token_idx, sc, counts, e, rpad, a1)
    used = (counts.cpu() + 127) // 128 * 128
    assert torch.equal(qt1[:, :int(used.sum())], qt2[:, :int(used.sum())])
    full = (counts > 0)
    assert torch.equal(st1[full], st2[full])


FP8_LAYER_CASES = {
    "shared_sigmoid": dict(bs=2, slen=512, dim=512, experts=16, top_k=4, hidden=256, shared_hidden=256),
    "no_shared_softmax": dict(bs=1, slen=768, dim=768, experts=8, top_k=2, hidden=512, shared_hidden=0,
                              score_func="softmax", route_norm=False, route_scale=1.0),
}


@pytest.mark.parametrize("name", list(FP8_LAYER_CASES))
def test_fp8_layer_fused_permute_matches_separate_ops(dev, name):
    """MoE with fp8 experts and the score before them: the fused op (moe_core_fp8,
    taken with MoE.fuse_fp8_permute: the permute inside the token quantizers, the
    combine's gather inside the backward's) gives the output, the input gradient
    and every parameter gradient bit-identical to permute -> experts -> combine."""
    banner(f"fp8 layer fused permute {name}")
    from tests.layer_util import LayerShape, build_layer

    sh = LayerShape(**FP8_LAYER_CASES[name], fp8=True)
    moe, x, gy = build_layer(sh, dev, seed=6)

    def run(fuse):
        moe.fuse_fp8_permute = fuse
        moe.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        assert (moe._fused_core(xx.view(-1, sh.dim)) is not None) == fuse
        out = moe(xx)
        out.backward(gy)
        torch.cuda.synchronize()
        return out.detach(), xx.grad, {n: p.grad.clone() for n, p in moe.named_parameters()}

    out_s, gx_s, gp_s = run(False)
    out_f, gx_f, gp_f = run(True)
    assert torch.equal(out_f, out_s)
    assert torch.equal(gx_f, gx_s)
    assert gp_f.keys() == gp_s.keys()
    for n in gp_s:
        assert torch.equal(gp_f[n], gp_s[n]), n
    print(f"[case] {name}: out, grad_x and {len(gp_s)} parameter gradients identical", flush=True)
