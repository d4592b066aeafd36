"""MXFP8 grouped SwiGLU experts on the GPU.

Parity is unpinned against the reference (its MXFP8 path is torchao's
MXFP8TrainingOpConfig, absent here); the kernels are checked against the
oracle's restatement of that recipe (quant_mxfp8, _mx_mm, experts_mxfp8_*),
which tests/test_oracle.py pins on the CPU, and against the bf16 experts:
  * quantizers: e4m3 bytes and e8m0 scales bit-exact vs the oracle, including
    blocks of zeros, blocks too small for any scale (e == 0) and wide dynamic
    ranges;
  * each MXFP8 GEMM entry point, fed the oracle's own quantized operands:
    normwise relative error <= 1e-2 (only the fp32 summation order differs);
    scale blocks the kernels must not read are poisoned with NaN (0xff);
  * the chained op (fwd + bwd): <= 5e-2 vs the emulation and <= 0.1 vs the
    fp32 reference on the bf16 inputs.
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
NAN_E8M0 = 255


def _rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def _u8(q):
    return q.view(torch.uint8).contiguous()


def _tokens_t(t, segs, rpad):
    """Oracle token-transposed layout: q [C, rpad] with 128-aligned zero-padded
    groups, scales [rpad / 32, C] k-block major (NaN where no group writes)."""
    c = t.shape[1]
    q = torch.zeros(c, rpad, dtype=torch.uint8)
    sc = torch.full((rpad // 32, c), NAN_E8M0, dtype=torch.uint8)
    per, pstart = [], 0
    for s0, n in segs:
        if n:
            qq, ss = R.quant_mxfp8(R._pad_tokens(t[s0:s0 + n].t(), 128))
            npad = qq.shape[1]
            q[:, pstart:pstart + npad] = qq.view(torch.uint8)
            sc[pstart // 32:pstart // 32 + npad // 32] = ss.t()
            per.append((qq, ss))
        else:
            per.append(None)
        pstart += (n + 127) // 128 * 128
    return q, sc, per


def test_mxfp8_quantizers_bit_exact(dev):
    banner("mxfp8 quantizers")
    from torchtitan_amd import _lib, ops

    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(300, 512, generator=g)
         * torch.exp(torch.randn(300, 16, generator=g) * 4).repeat_interleave(32, 1)).bfloat16()
    x[7] = 0                      # all-zero blocks: e = 0
    x[9, 64:96] = 2.0 ** -121     # amax / 448 below 2^-127: e = 0, multiplier 1
    x[11, 0:32] = 448.0           # exact power-of-two boundary
    x[11, 32:64] = 450.0
    q, s = ops._mx_quant_rows(x.to(dev), 512)
    rq, rs = R.quant_mxfp8(x)
    assert torch.equal(s.cpu(), rs), "e8m0 scales differ"
    assert torch.equal(q.cpu(), rq.view(torch.uint8)), "MX bytes differ"
    # columns, transposed and strided: w [E, A, B] -> rows (e, b) of A values
    e, a, b = 3, 256, 128
    w = (torch.randn(e, a, b, generator=g) * torch.exp(torch.randn(e, a, 1, generator=g) * 2)).bfloat16()
    qt = torch.zeros(e, b, 2 * a, dtype=torch.uint8, device=dev)        # a row stride of 2a: the [E, D, 2H] layout
    stt = torch.zeros(e, b, 2 * a // 32, dtype=torch.uint8, device=dev)
    wd = w.to(dev)
    _lib.call("moe_mxfp8_quant_cols_t", wd.data_ptr(), e, a, b, qt.data_ptr() + a, b * 2 * a, 2 * a,
              stt.data_ptr() + a // 32, b * (2 * a // 32), 2 * a // 32, st)
    qt, stt = qt.cpu(), stt.cpu()
    for i in range(e):
        rq, rs = R.quant_mxfp8(w[i].t())
        assert torch.equal(qt[i, :, a:], rq.view(torch.uint8))
        assert torch.equal(stt[i, :, a // 32:], rs)
        assert torch.count_nonzero(qt[i, :, :a]) == 0 and torch.count_nonzero(stt[i, :, :a // 32]) == 0
    # token groups, transposed and 32-padded, k-block-major scales
    counts = torch.tensor([5, 0, 33, 32, 1, 64, 200], dtype=torch.int64)
    r, c = int(counts.sum()), 128
    xt = torch.randn(r, c, generator=g).bfloat16()
    rpad = ops._mx_padded_rows(r, len(counts))
    assert rpad % 128 == 0 and rpad >= r + 127 * len(counts)
    q2, s2 = ops._mx_quant_tokens_t(xt.to(dev), counts.to(dev), len(counts), rpad)
    q2, s2 = q2.cpu(), s2.cpu()
    segs = [(int(counts[:i].sum()), int(n)) for i, n in enumerate(counts)]
    rq2, rs2, _ = _tokens_t(xt, segs, rpad)
    used = sum((n + 127) // 128 * 128 for _, n in segs)
    assert torch.equal(q2[:, :used], rq2[:, :used])
    assert torch.equal(s2[:used // 32], rs2[:used // 32])
    # dual: one read, both layouts
    qr, sr, qt, st_ = ops._mx_dual_tokens(xt.to(dev), counts.to(dev), len(counts), rpad)
    rqr, rsr = R.quant_mxfp8(xt)
    assert torch.equal(qr.cpu(), rqr.view(torch.uint8)) and torch.equal(sr.cpu(), rsr)
    assert torch.equal(qt.cpu()[:, :used], rq2[:, :used]) and torch.equal(st_.cpu()[:used // 32], rs2[:used // 32])
    w1 = (torch.randn(e, 2 * a, b, generator=g) * torch.exp(torch.randn(e, 2 * a, 1, generator=g))).bfloat16()
    w3 = torch.randn(e, 2 * a, b, generator=g).bfloat16()
    w2 = torch.randn(e, b, 2 * a, generator=g).bfloat16()
    outs = ops._mx_weights(w1.to(dev), w2.to(dev), w3.to(dev), True)
    qw1, sw1, qw3, sw3, qw2, sw2, qw2t, sw2t, qw13t, sw13t = (t.cpu() for t in outs)
    hh_ = 2 * a
    for w, q_, s_ in ((w1, qw1, sw1), (w3, qw3, sw3), (w2, qw2, sw2)):
        rq, rs = R.quant_mxfp8(w.reshape(-1, w.shape[-1]))
        assert torch.equal(q_, rq.view(torch.uint8)) and torch.equal(s_, rs)
    for i in range(e):
        rq, rs = R.quant_mxfp8(w2[i].t())
        assert torch.equal(qw2t[i], rq.view(torch.uint8)) and torch.equal(sw2t[i], rs)
        for half, w in ((0, w1), (1, w3)):
            rq, rs = R.quant_mxfp8(w[i].t())
            assert torch.equal(qw13t[i][:, half * hh_:(half + 1) * hh_], rq.view(torch.uint8))
            assert torch.equal(sw13t[i][:, half * hh_ // 32:(half + 1) * hh_ // 32], rs)



@pytest.mark.parametrize("width", [192, 320, 384])
def test_mxfp8_transposing_quantizers_slab_widths(dev, width):
    """The MXFP8 transposing and dual quantizers at widths that take 64-column
    slabs (192, 320) and 128-column ones (384): bit-exact against the oracle."""
    banner(f"mxfp8 transposing quantizers width={width}")
    from torchtitan_amd import _lib, ops
    g = torch.Generator().manual_seed(width)
    st = torch.cuda.current_stream().cuda_stream
    e, a = 3, 256
    w = torch.randn(e, a, width, generator=g).bfloat16()
    qr = torch.empty(e * a, width, dtype=torch.uint8, device=dev)
    sr = torch.empty(e * a, width // 32, dtype=torch.uint8, device=dev)
    qt = torch.empty(e, width, a, dtype=torch.uint8, device=dev)
    stt = torch.empty(e, width, a // 32, dtype=torch.uint8, device=dev)
    _lib.call("moe_mxfp8_quant_dual_cols", w.to(dev).data_ptr(), e, a, width, qr.data_ptr(), sr.data_ptr(),
              qt.data_ptr(), width * a, a, stt.data_ptr(), width * (a // 32), a // 32, st)
    rq, rs = R.quant_mxfp8(w.reshape(-1, width))
    assert torch.equal(qr.cpu(), rq.view(torch.uint8)) and torch.equal(sr.cpu(), rs)
    for i in range(e):
        rq, rs = R.quant_mxfp8(w[i].t())
        assert torch.equal(qt[i].cpu(), rq.view(torch.uint8)) and torch.equal(stt[i].cpu(), rs)
    counts = torch.tensor([5, 0, 300, 32, 1], dtype=torch.int64)
    r = int(counts.sum())
    xt = torch.randn(r, width, generator=g).bfloat16()
    rpad = ops._mx_padded_rows(r, len(counts))
    segs = [(int(counts[:i].sum()), int(n)) for i, n in enumerate(counts)]
    rq2, rs2, _ = _tokens_t(xt, segs, rpad)
    used = sum((n + 127) // 128 * 128 for _, n in segs)
    q2, s2 = ops._mx_quant_tokens_t(xt.to(dev), counts.to(dev), len(counts), rpad)
    assert torch.equal(q2.cpu()[:, :used], rq2[:, :used]) and torch.equal(s2.cpu()[:used // 32], rs2[:used // 32])
    dqr, dsr, dqt, dst = ops._mx_dual_tokens(xt.to(dev), counts.to(dev), len(counts), rpad)
    rqr, rsr = R.quant_mxfp8(xt)
    assert torch.equal(dqr.cpu(), rqr.view(torch.uint8)) and torch.equal(dsr.cpu(), rsr)
    assert torch.equal(dqt.cpu()[:, :used], rq2[:, :used]) and torch.equal(dst.cpu()[:used // 32], rs2[:used // 32])

# experts, D, H, rows per expert: ragged with empty experts; tall experts over several
# 256-row m-tiles with partial last tiles; single-row and tile-edge groups
GEMM_SHAPES = {
    "ragged_e6_d256_h256": (6, 256, 256, [40, 0, 130, 17, 64, 3]),
    "tall_e3_d512_h768": (3, 512, 768, [700, 0, 517]),
    "edges_e5_d768_h256": (5, 768, 256, [1, 255, 257, 0, 390]),
}


@pytest.mark.parametrize("shape", list(GEMM_SHAPES))
def test_mxfp8_gemm_entry_points_match_emulation(dev, shape):
    """Every MXFP8 GEMM kernel against R._mx_mm on identical quantized operands."""
    banner("mxfp8 GEMM entry points")
    from torchtitan_amd import _lib, ops

    e, d, h, counts = GEMM_SHAPES[shape]
    gen = torch.Generator().manual_seed(2)
    r = sum(counts)
    cnt = torch.tensor(counts, dtype=torch.int64)

    def rnd(*shape, scale=1.0):
        # block-varying magnitudes so that neighbouring scales differ
        t = torch.randn(*shape, generator=gen) * scale
        return (t * torch.exp2(torch.randint(-3, 4, (*shape[:-1], shape[-1] // 32), generator=gen).float()
                               ).repeat_interleave(32, -1)).bfloat16()
    x = rnd(r, d)
    w1, w3 = rnd(e, h, d, scale=0.05), rnd(e, h, d, scale=0.05)
    w2 = rnd(e, d, h, scale=0.05)
    dy = rnd(r, d)
    gg, uu = rnd(r, h), rnd(r, h)
    dgu = rnd(r, 2 * h)
    hh = rnd(r, h)
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
    qx, sx = R.quant_mxfp8(x)
    qw1, sw1 = R.quant_mxfp8(w1)
    qw3, sw3 = R.quant_mxfp8(w3)
    g_, u_, h_ = (torch.empty(r, h, dtype=torch.bfloat16, device=dev) for _ in range(3))
    _lib.call("moe_mxfp8_gemm_gate_up", P(_u8(qx)), P(sx), P(_u8(qw1)), P(sw1), P(_u8(qw3)), P(sw3), cd.data_ptr(),
              r, e, d, h, g_.data_ptr(), u_.data_ptr(), h_.data_ptr(), st)
    eg = per_expert(lambda i, sl: R._mx_mm(qx[sl], sx[sl], qw1[i], sw1[i]).bfloat16())
    eu = per_expert(lambda i, sl: R._mx_mm(qx[sl], sx[sl], qw3[i], sw3[i]).bfloat16())
    print(f"[case] gate_up g {_rel(g_, eg):.2e} u {_rel(u_, eu):.2e}", flush=True)
    assert _rel(g_, eg) <= GEMM_TOL and _rel(u_, eu) <= GEMM_TOL
    assert _rel(h_, F.silu(eg) * eu) <= GEMM_TOL
    # the epilogue's h from its own g and u is torch's silu(g) * u bit for bit
    assert torch.equal(h_, F.silu(g_) * u_)
    # down
    qh, sh = R.quant_mxfp8(hh)
    qw2, sw2 = R.quant_mxfp8(w2)
    y_ = torch.empty(r, d, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_mxfp8_gemm_down", P(_u8(qh)), P(sh), P(_u8(qw2)), P(sw2), cd.data_ptr(), r, e, d, h,
              y_.data_ptr(), st)
    ey = per_expert(lambda i, sl: R._mx_mm(qh[sl], sh[sl], qw2[i], sw2[i]).bfloat16())
    print(f"[case] down {_rel(y_, ey):.2e}", flush=True)
    assert _rel(y_, ey) <= GEMM_TOL
    # bwd dgu (dh checked through du = dh * bf16(silu(g)))
    qdy, sdy = R.quant_mxfp8(dy)
    qw2t, sw2t = zip(*(R.quant_mxfp8(w2[i].t()) for i in range(e)))
    qw2t, sw2t = torch.stack(qw2t), torch.stack(sw2t)
    dgu_ = torch.empty(r, 2 * h, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_mxfp8_gemm_bwd_dgu", P(_u8(qdy)), P(sdy), P(_u8(qw2t)), P(sw2t), P(gg), P(uu), cd.data_ptr(), r,
              e, d, h, dgu_.data_ptr(), st)
    dh = per_expert(lambda i, sl: R._mx_mm(qdy[sl], sdy[sl], qw2t[i], sw2t[i]).bfloat16())
    assert _rel(dgu_[:, h:], dh * F.silu(gg)) <= GEMM_TOL
    assert _rel(dgu_[:, :h], torch.ops.aten.silu_backward(dh * uu, gg)) <= GEMM_TOL
    # bwd dx: [dg | du] blocked along 2H, w1^T and w3^T side by side
    qdgu, sdgu = R.quant_mxfp8(dgu)
    qw1t, sw1t = zip(*(R.quant_mxfp8(w1[i].t()) for i in range(e)))
    qw3t, sw3t = zip(*(R.quant_mxfp8(w3[i].t()) for i in range(e)))
    qw13t = torch.cat([torch.stack(qw1t).view(torch.uint8), torch.stack(qw3t).view(torch.uint8)], dim=2)
    sw13t = torch.cat([torch.stack(sw1t), torch.stack(sw3t)], dim=2)
    dx_ = torch.empty(r, d, dtype=torch.bfloat16, device=dev)
    _lib.call("moe_mxfp8_gemm_bwd_dx", P(_u8(qdgu)), P(sdgu), P(qw13t), P(sw13t), cd.data_ptr(), r, e, d, h,
              dx_.data_ptr(), st)
    hb = h // 32
    edx = per_expert(lambda i, sl: R._mx_mm(qdgu[sl, :h], sdgu[sl, :hb], qw1t[i], sw1t[i]).bfloat16()
                     + R._mx_mm(qdgu[sl, h:], sdgu[sl, hb:], qw3t[i], sw3t[i]).bfloat16())
    print(f"[case] dx {_rel(dx_, edx):.2e}", flush=True)
    assert _rel(dx_, edx) <= GEMM_TOL
    # bwd dw13 / dw2 from token-transposed, 32-padded operands
    rpad = ops._mx_padded_rows(r, e)
    qdgut, sdgut, ldgu = _tokens_t(dgu, segs, rpad)
    qxt, sxt, lx = _tokens_t(x, segs, rpad)
    dw1_, dw3_ = torch.empty_like(w1, device=dev), torch.empty_like(w3, device=dev)
    _lib.call("moe_mxfp8_gemm_bwd_dw13", P(qdgut), P(sdgut), P(qxt), P(sxt), cd.data_ptr(), r, rpad, e, d, h,
              dw1_.data_ptr(), dw3_.data_ptr(), st)
    qdyt, sdyt, ldy = _tokens_t(dy, segs, rpad)
    qht, sht, lh = _tokens_t(hh, segs, rpad)
    dw2_ = torch.empty_like(w2, device=dev)
    _lib.call("moe_mxfp8_gemm_bwd_dw2", P(qdyt), P(sdyt), P(qht), P(sht), cd.data_ptr(), r, rpad, e, d, h,
              dw2_.data_ptr(), st)
    for i, (s0, n) in enumerate(segs):
        if n == 0:
            for t in (dw1_, dw2_, dw3_):
                assert torch.count_nonzero(t[i]) == 0
            continue
        (qa, sa), (qb, sb) = ldgu[i], lx[i]
        edw = R._mx_mm(qa, sa, qb, sb).bfloat16()  # [2H, D]
        errs = (_rel(dw1_[i], edw[:h]), _rel(dw3_[i], edw[h:]))
        (qa, sa), (qb, sb) = ldy[i], lh[i]
        errs += (_rel(dw2_[i], R._mx_mm(qa, sa, qb, sb).bfloat16()),)
        print(f"[case] expert {i} ({n} tokens) dw1/dw3/dw2 " + " ".join(f"{v:.2e}" for v in errs), flush=True)
        assert max(errs) <= GEMM_TOL, errs


CASES = {
    "ragged_e8": (8, 256, 512, [37, 0, 130, 16, 255, 1, 64, 100]),
    "e16_d512_h256": (16, 512, 256, [96, 81, 0, 0, 200, 17, 33, 64, 128, 5, 70, 90, 300, 2, 0, 40]),
}


@pytest.mark.parametrize("for_backward", [True, False])
@pytest.mark.parametrize("name", list(CASES))
def test_mxfp8_grouped_swiglu_fwd_bwd(dev, name, for_backward):
    """for_backward=True: the forward's dual quantizers keep the transposed
    layouts for the backward; False: the backward quantizes them itself."""
    e, d, h, counts = CASES[name]
    banner(f"mxfp8 grouped swiglu {name} for_backward={for_backward}")
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
    y, gg, uu, hh, *_ = ops.grouped_swiglu_mxfp8(xs, a, b, c, cnt.to(dev), for_backward)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    ey, eg, eu, eh = R.experts_mxfp8_forward(w1, w2, w3, x, cnt)
    edx, edw1, edw2, edw3 = R.experts_mxfp8_backward(w1, w2, w3, x, cnt, eg, eu, eh, dy)
    errs = {"y": _rel(y, ey), "g": _rel(gg, eg), "h": _rel(hh, eh), "dx": _rel(xs.grad, edx),
            "dw1": _rel(a.grad, edw1), "dw2": _rel(b.grad, edw2), "dw3": _rel(c.grad, edw3)}
    print(f"[case] {name} vs MXFP8 emulation: {errs}", flush=True)
    assert all(v <= EMU_TOL for v in errs.values()), errs
    for i, n in enumerate(counts):
        if n == 0:
            for t in (a.grad, b.grad, c.grad):
                assert torch.count_nonzero(t[i]) == 0
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


def test_mxfp8_quantizers_nan_elements(dev):
    """A NaN element quantizes to 0x7f and sends only its own wave (row-wise) or
    LDS tile (transposed) to the software conversion: every 32-block without a
    NaN still matches the oracle bit for bit (the NaN's own block is not
    compared: its scale skips the NaN here, torch's amax propagates it)."""
    banner("mxfp8 quantizers with NaN elements")
    from torchtitan_amd import ops

    g = torch.Generator().manual_seed(6)
    x = torch.randn(256, 128, generator=g).bfloat16()
    x[13, 5] = float("nan")
    x[200, 70] = float("nan")
    q, s = ops._mx_quant_rows(x.to(dev), 128)
    q, s = q.cpu(), s.cpu()
    rq, rs = R.quant_mxfp8(x)
    rq = rq.view(torch.uint8)
    assert q[13, 5].item() == 0x7F and q[200, 70].item() == 0x7F
    blk = torch.ones(256, 4, dtype=torch.bool)
    blk[13, 0] = False
    blk[200, 2] = False
    assert torch.equal(s[blk], rs[blk])
    el = blk.repeat_interleave(32, dim=1)
    assert torch.equal(q[el], rq[el])
    # token groups, transposed (and the dual kernel's row-wise layout from the same read)
    counts = torch.tensor([100, 0, 156], dtype=torch.int64)
    rpad = ops._mx_padded_rows(256, 3)
    segs = [(0, 100), (100, 0), (100, 156)]
    rq2, rs2, _ = _tokens_t(x, segs, rpad)
    for qt, st_ in (ops._mx_quant_tokens_t(x.to(dev), counts.to(dev), 3, rpad),
                    ops._mx_dual_tokens(x.to(dev), counts.to(dev), 3, rpad)[2:]):
        qt, st_ = qt.cpu(), st_.cpu()
        assert qt[5, 13].item() == 0x7F and qt[70, 128 + 100].item() == 0x7F
        ok = torch.ones(128, rpad // 32, dtype=torch.bool)  # (column, k-block) pairs without a NaN
        ok[5, 0] = False
        ok[70, (128 + 100) // 32] = False
        used = (128 + 256) // 32
        ok[:, used:] = False
        assert torch.equal(st_.t()[ok], rs2.t()[ok])
        el = ok.repeat_interleave(32, dim=1)
        assert torch.equal(qt[el], rq2[el])
    qr, sr, _, _ = ops._mx_dual_tokens(x.to(dev), counts.to(dev), 3, rpad)
    qr, sr = qr.cpu(), sr.cpu()
    assert qr[13, 5].item() == 0x7F and qr[200, 70].item() == 0x7F
    assert torch.equal(sr[blk], rs[blk])
    el = blk.repeat_interleave(32, dim=1)
    assert torch.equal(qr[el], rq[el])


@pytest.mark.parametrize("cols", [256, 192])
@pytest.mark.parametrize("scaled", [True, False])
def test_mxfp8_gathering_token_quantizer_matches_permute_then_quantize(dev, cols, scaled):
    """moe_mxfp8_quant_dual_tokens_gather reads the routed rows x[token_idx]
    (* score, rounded to bf16) in place: all four layouts byte-identical to the
    permute op's output fed to moe_mxfp8_quant_dual_tokens (ragged groups, an
    empty expert, 64-column slabs when the width is no multiple of 128)."""
    banner(f"mxfp8 gathering token quantizer cols={cols} scaled={scaled}")
    from torchtitan_amd import ops

    g = torch.Generator().manual_seed(11)
    n, e, k = 300, 8, 2
    x = (torch.randn(n, cols, generator=g) * 3).bfloat16().to(dev)
    logits = torch.randn(n, e, generator=g)
    logits[:, 3] = -1e9  # expert 3 receives no token
    top, idx = logits.topk(k, dim=1)
    top = top.sigmoid().to(dev)
    scores_sorted, token_idx, counts, _offs, slot_pos, tok_pos = ops.reorder(top, idx.to(dev), e)
    assert counts[3].item() == 0
    r = n * k
    rpad = ops._mx_padded_rows(r, e)
    routed = ops.permute(x, slot_pos, tok_pos, scores_sorted if scaled else None)
    want = ops._mx_dual_tokens(routed, counts, e, rpad)
    got = ops._mx_dual_tokens_gather(x, token_idx, scores_sorted if scaled else None, counts, e, rpad)
    torch.cuda.synchronize()
    for name, a, b in zip(("q_rows", "s_rows", "q_t", "s_t"), got, want):
        assert torch.equal(a, b), name


LAYER_CASES = {
    "shared_sigmoid": dict(bs=2, slen=512, dim=512, experts=16, top_k=4, hidden=256, shared_hidden=256),
    "no_shared_softmax": dict(bs=1, slen=768, dim=768, experts=8, top_k=2, hidden=512, shared_hidden=0,
                              score_func="softmax", route_norm=False, route_scale=1.0),
}


@pytest.mark.parametrize("name", list(LAYER_CASES))
def test_mxfp8_layer_fused_permute_matches_separate_ops(dev, name):
    """MoE with MXFP8 experts and the score before them: the fused op
    (moe_core_mxfp8: permute inside the token quantizer, the combine's gather
    inside the backward's) gives the output, the input gradient and every
    parameter gradient bit-identical to permute -> experts -> combine."""
    banner(f"mxfp8 layer fused permute {name}")
    from tests.layer_util import LayerShape, build_layer

    sh = LayerShape(**LAYER_CASES[name], mxfp8=True)
    moe, x, gy = build_layer(sh, dev, seed=5)

    def run(fuse):
        moe.fuse_permute_into_quantizers = fuse
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


def test_mxfp8_layer_hook_on_experts_keeps_the_experts_call(dev):
    """The fused MXFP8 op reads the expert weights without calling the experts
    module; a forward hook on that module turns the fusion off, so the hook sees
    the call, and the results are those of the separate ops."""
    banner("mxfp8 layer with a hook on the experts")
    from tests.layer_util import LayerShape, build_layer

    sh = LayerShape(**LAYER_CASES["shared_sigmoid"], mxfp8=True)
    moe, x, gy = build_layer(sh, dev, seed=6)
    xx = x.clone().requires_grad_(True)
    assert moe._fused_core(xx.view(-1, sh.dim)) is not None
    moe.zero_grad(set_to_none=True)
    ref = moe(xx)
    ref.backward(gy)
    gx_ref = xx.grad.clone()
    seen = []
    handle = moe.experts.register_forward_hook(lambda m, a, o: seen.append(a[0].shape))
    try:
        assert moe._fused_core(xx.view(-1, sh.dim)) is None
        moe.zero_grad(set_to_none=True)
        xx.grad = None
        out = moe(xx)
        out.backward(gy)
        torch.cuda.synchronize()
    finally:
        handle.remove()
    assert seen == [(sh.bs * sh.slen * sh.top_k, sh.dim)]
    assert torch.equal(out, ref) and torch.equal(xx.grad, gx_ref)
