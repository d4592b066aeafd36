"""Benchmark of the MI355X MoE layer hot path (forward + backward of one MoE layer).

Workload (default): the Kimi-Linear-48B-A3B-shape MoE layer, bf16 — dim 2304,
256 routed experts, top-8 sigmoid scores + per-expert bias ~ U(-0.01, 0.01),
route norm on, route scale 2.5, SwiGLU experts with hidden 1024 plus one shared
SwiGLU expert with hidden 1024, 16384 tokens (batch 4 x seq 4096), x ~ N(0,1),
weights N(0, 0.02), backward seeded with g ~ N(0,1). Synthetic data and
random-init weights; everything is resident in HBM before timing starts.

A step is MoE.forward + backward of that layer (torchtitan/models/common/moe.py:380-477
and its autograd). The JSON line reports routed tokens/s (N*K per step), the
grouped-GEMM TFLOP/s over the six grouped GEMM kernels, per-kernel HIP-event
timings taken inside the timed steps, the roofline of the dominant kernel, and
the reference's CPU MoE path (the oracle's op-for-op restatement) timed on a
bounded token sample on this host's cores.

The timed steps run uninstrumented (that time gives `value`); a second pass of
the same number of steps brackets every C-ABI launch with HIP events on its
stream for the per-kernel table and the roofline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--workload kimi|dsv3|zipf|kimi_fp8|kimi_mxfp8|gptoss_20b|c1|c1_grouped]
                       [--no-cpu-baseline] [--cpu-tokens N] [--gemm-ceiling] [--mover-ceiling]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from types import SimpleNamespace

import torch

# one GPU: no pipeline, context or expert parallelism
_NO_PARALLEL = SimpleNamespace(pp_enabled=False, cp_enabled=False, ep_enabled=False)

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0  # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E

WORKLOADS = {
    # name: dict of layer shape and routing settings
    "kimi": dict(
        desc="Kimi-Linear-48B-A3B-shape MoE layer",
        bs=4, slen=4096, dim=2304, experts=256, top_k=8, hidden=1024, shared_hidden=1024,
        score_func="sigmoid", route_norm=True, route_scale=2.5, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.01, zipf=None,
    ),
    "dsv3": dict(
        desc="DeepSeek-V3-style group-limited MoE layer",
        bs=1, slen=8192, dim=7168, experts=256, top_k=8, hidden=2048, shared_hidden=2048,
        score_func="sigmoid", route_norm=True, route_scale=2.5, groups=8, limited=4,
        score_before=False, std=0.006, bias=0.01, zipf=None,
    ),
    "zipf": dict(
        desc="Kimi-shape MoE layer with Zipf(1.2)-skewed expert load",
        bs=8, slen=4096, dim=2304, experts=256, top_k=8, hidden=1024, shared_hidden=1024,
        score_func="sigmoid", route_norm=True, route_scale=2.5, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.01, zipf=1.2,
    ),
    "kimi_32k": dict(
        desc="Kimi-shape MoE layer at 32768 tokens, bf16 (the fp8 workloads' token count)",
        bs=8, slen=4096, dim=2304, experts=256, top_k=8, hidden=1024, shared_hidden=1024,
        score_func="sigmoid", route_norm=True, route_scale=2.5, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.01, zipf=None,
    ),
    "kimi_fp8": dict(
        desc="Kimi-shape MoE layer with fp8 e4m3 grouped GEMMs",
        bs=8, slen=4096, dim=2304, experts=256, top_k=8, hidden=1024, shared_hidden=1024,
        score_func="sigmoid", route_norm=True, route_scale=2.5, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.01, zipf=None, fp8=True,
    ),
    "kimi_mxfp8": dict(
        desc="Kimi-shape MoE layer with MXFP8 (block-32 e8m0, RCEIL) grouped GEMMs",
        bs=8, slen=4096, dim=2304, experts=256, top_k=8, hidden=1024, shared_hidden=1024,
        score_func="sigmoid", route_norm=True, route_scale=2.5, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.01, zipf=None, mxfp8=True,
    ),
    "c1": dict(
        desc="tiny fp32 MoE layer, fp32 experts (the for-loop path)",
        bs=2, slen=2048, dim=256, experts=8, top_k=2, hidden=512, shared_hidden=0,
        score_func="softmax", route_norm=False, route_scale=1.0, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.0, zipf=None, fp32=True, grouped=False,
    ),
    "c1_grouped": dict(
        desc="tiny fp32 MoE layer, bf16 grouped-mm experts (use_grouped_mm=True)",
        bs=2, slen=2048, dim=256, experts=8, top_k=2, hidden=512, shared_hidden=0,
        score_func="softmax", route_norm=False, route_scale=1.0, groups=None, limited=None,
        score_before=True, std=0.02, bias=0.0, zipf=None, fp32=True, grouped=True,
    ),
    "gptoss_20b": dict(
        desc="gpt-oss-20b-shape MoE layer (biased clamped-SwiGLU experts, biased softmax gate)",
        bs=4, slen=4096, dim=2880, experts=32, top_k=4, hidden=2880, shared_hidden=0,
        score_func="softmax", route_norm=True, route_scale=1.0, groups=None, limited=None,
        score_before=False, std=0.02, bias=0.01, zipf=None, gptoss=True,
    ),
}

PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 MFMA

GEMM_ENTRIES = tuple(f"moe_{kind}_{m}" for kind in ("grouped_gemm", "fp8_gemm", "mxfp8_gemm", "grouped_gemm_oss",
                                                   "grouped_gemm_f32")
                     for m in ("gate_up", "down", "bwd_dgu", "bwd_dx", "bwd_dw13", "bwd_dw1", "bwd_dw2", "bwd_dw"))


def kernel_work(name: str, w: dict) -> tuple[str, float]:
    """Algorithmic work of one launch of C-ABI entry `name` for workload `w`:
    ("mfma", flops) for the grouped GEMMs, ("hbm", bytes) for the data movers.
    Bytes count each tensor element the launch must read or write once."""
    n = w["bs"] * w["slen"]
    d, e, k, h = w["dim"], w["experts"], w["top_k"], w["hidden"]
    r = n * k
    b = 4 if w.get("fp32") else 2  # row bytes per element (fp32 activations on the c1 workloads)
    sb = w.get("score_before", True)
    # bwd_dw (fp32 kernels) is one launch per weight: 2 R D H each
    flops = {"gate_up": 4, "down": 2, "bwd_dgu": 2, "bwd_dx": 4, "bwd_dw13": 4, "bwd_dw1": 4, "bwd_dw2": 2,
             "bwd_dw": 2}
    for kind in ("moe_grouped_gemm_oss_", "moe_grouped_gemm_f32_", "moe_grouped_gemm_", "moe_fp8_gemm_",
                 "moe_mxfp8_gemm_"):
        if name.startswith(kind) and name[len(kind):] in flops:
            return "mfma", float(flops[name[len(kind):]] * r * d * h)
    nbytes = {
        # logits [N,E] f32 read; scores [N,E] f32, top scores f32 and ids i64 [N,K] written
        "moe_router_fwd": 4 * n * e + 4 * n * e + 12 * n * k,
        "moe_histogram": 8 * n * k + 8 * e,
        # ids read twice (histogram + scatter), sorted scores/token ids and two int32 maps written
        "moe_reorder": 16 * n * k + 4 * n * k + 4 * r + 8 * r + 8 * n * k,
        # x read once, K copies written, slot map read (+ sorted scores when the score
        # multiplies the expert inputs)
        "moe_permute": n * d * b + r * d * b + 4 * n * k + (4 * r if sb else 0),
        # routed rows + shared rows read, out written, tok map read (+ sorted scores when the
        # score multiplies the expert outputs)
        "moe_combine": r * d * b + 2 * n * d * b + 4 * n * k + (0 if sb else 4 * r),
        # score before the experts: the gather grad_out[token] into K copies; after them:
        # grad_out and the routed rows read, the scaled copies and score gradients written
        "moe_combine_bwd": (n * d * b + r * d * b + 4 * n * k) if sb else
                           (n * d * b + 2 * r * d * b + 4 * n * k + 8 * r),
        # grad_routed read, grad_x written (+ x read and score gradients written when the
        # score multiplies the expert inputs)
        "moe_permute_bwd": (r * d * b + 2 * n * d * b + 4 * n * k + 8 * r) if sb else
                           (r * d * b + n * d * b + 4 * n * k),
        "moe_reorder_bwd": 4 * r + 4 * n * k + 4 * n * k,
        "moe_router_bwd": 4 * n * k + 8 * n * k + 4 * n * e + 4 * n * e,
    }
    # the quantizers run on tensors of several sizes per step: bytes per launch come
    # from the launch's own arguments (launch_bytes)
    return "hbm", (float(nbytes[name]) if name in nbytes else None)


def launch_bytes(name: str, a: tuple) -> float | None:
    """Algorithmic bytes of one quantizer launch from its C-ABI arguments: the bf16
    input read once, the fp8 codes and scales written once (fp32 scales per row, per
    column or per (expert, column); e8m0 scales per 32 elements for MXFP8)."""
    mx = 1.0 + 1.0 / 32.0
    if name == "moe_fp8_quant_rows":
        rows, cols = a[1], a[2]
        return 3.0 * rows * cols + 4.0 * rows
    if name == "moe_fp8_quant_cols_t":
        e, ra, cb = a[1], a[2], a[3]
        return 3.0 * e * ra * cb + 4.0 * e * cb
    if name == "moe_fp8_quant_rows_colamax":  # + the [E, b] column amax written
        e, ra, cb = a[1], a[2], a[3]
        return 3.0 * e * ra * cb + 4.0 * e * ra + 4.0 * e * cb
    if name == "moe_fp8_quant_cols_t_amax":  # the column amax read instead of found
        e, ra, cb = a[2], a[3], a[4]
        return 3.0 * e * ra * cb + 8.0 * e * cb
    if name == "moe_swiglu_fwd":  # a1, a3 read, h written
        return 3.0 * a[2] * a[3] * (2 if a[4] == 0 else 4)
    if name == "moe_swiglu_bwd":  # dh, a1, a3 read, dg and du written
        return 5.0 * a[3] * a[4] * (2 if a[5] == 0 else 4)
    if name == "moe_gate_grad_split3":  # fp32 gradient read, three bf16 terms written
        return 10.0 * a[1] * a[2]
    if name == "moe_gate_dw_reduce":  # fp32 partials read, bf16 dW written
        return 12.0 * a[1] * a[2] * a[3] + 2.0 * a[2] * a[3]
    if name == "moe_fp8_quant_tokens_t":
        rows, e, cols, padded = a[2], a[3], a[4], a[5]
        return 2.0 * rows * cols + 1.0 * padded * cols + 4.0 * e * cols + 8.0 * e
    if name == "moe_fp8_quant_rows_groupamax":  # + the [E, cols] group amax written
        rows, e, cols, pieces = a[2], a[3], a[4], a[5]
        return 3.0 * rows * cols + 4.0 * rows * pieces + 4.0 * e * cols + 8.0 * e
    if name == "moe_fp8_quant_tokens_t_amax":  # the group amax read instead of found
        rows, e, cols, padded = a[3], a[4], a[5], a[6]
        return 2.0 * rows * cols + 1.0 * padded * cols + 8.0 * e * cols + 8.0 * e
    if name == "moe_fp8_quant_rows_groupamax_gather":  # + the row indices (and scores) read
        rows, e, cols = a[5], a[6], a[7]
        return 3.0 * rows * cols + 4.0 * rows + 4.0 * e * cols + 8.0 * e + (8.0 + (4.0 if a[3] else 0.0)) * rows
    if name == "moe_fp8_quant_tokens_t_amax_gather":
        rows, e, cols, padded = a[6], a[7], a[8], a[9]
        idx = (8.0 + (4.0 if a[3] else 0.0)) * rows
        return 2.0 * rows * cols + 1.0 * padded * cols + 8.0 * e * cols + 8.0 * e + idx
    if name == "moe_mxfp8_quant_rows":
        rows, cols = a[1], a[2]
        return 2.0 * rows * cols + mx * rows * cols
    if name == "moe_mxfp8_quant_cols_t":
        e, ra, cb = a[1], a[2], a[3]
        return 2.0 * e * ra * cb + mx * e * ra * cb
    if name == "moe_mxfp8_quant_dual_cols":
        e, ra, cb = a[1], a[2], a[3]
        return 2.0 * e * ra * cb + 2.0 * mx * e * ra * cb
    if name == "moe_mxfp8_quant_tokens_t":
        rows, e, cols, padded = a[2], a[3], a[4], a[5]
        return 2.0 * rows * cols + mx * padded * cols + 8.0 * e
    if name == "moe_mxfp8_quant_dual_tokens":
        rows, e, cols, padded = a[2], a[3], a[4], a[5]
        return 2.0 * rows * cols + mx * rows * cols + mx * padded * cols + 8.0 * e
    if name == "moe_mxfp8_quant_dual_tokens_gather":  # + the row indices (and scores) read
        rows, e, cols, padded = a[5], a[6], a[7], a[8]
        idx = (8.0 + (4.0 if a[3] else 0.0)) * rows
        return 2.0 * rows * cols + mx * rows * cols + mx * padded * cols + 8.0 * e + idx
    return None


def make_layer(w: dict, device: torch.device, seed: int):
    from torchtitan_amd import FeedForward, GroupedExperts, Linear, MoE, TokenChoiceTopKRouter
    from torchtitan_amd.gpt_oss import GptOssMoE

    d, e, h, hs = w["dim"], w["experts"], w["hidden"], w["shared_hidden"]
    cls = GptOssMoE if w.get("gptoss") else MoE
    cfg = cls.Config(
        num_experts=e,
        experts=GroupedExperts.Config(dim=d, hidden_dim=h, num_experts=e,
                                      use_grouped_mm=w.get("grouped", True)),
        router=TokenChoiceTopKRouter.Config(
            num_experts=e, gate=Linear.Config(in_features=d, out_features=e, bias=bool(w.get("gptoss"))),
            top_k=w["top_k"],
            score_func=w["score_func"], route_norm=w["route_norm"], route_scale=w["route_scale"],
            num_expert_groups=w["groups"], num_limited_groups=w["limited"],
        ),
        score_before_experts=w["score_before"],
        load_balance_coeff=1e-3,
        shared_experts=FeedForward.Config(
            w1=Linear.Config(in_features=d, out_features=hs),
            w2=Linear.Config(in_features=hs, out_features=d),
            w3=Linear.Config(in_features=d, out_features=hs),
        ) if hs else None,
    )
    with torch.device("meta"):
        moe = cfg.build()
    moe = moe.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    pdtype = torch.float32 if w.get("fp32") else torch.bfloat16
    with torch.no_grad():
        for name, p in moe.named_parameters():
            t = torch.empty(p.shape, dtype=torch.float32, device=device)
            if w.get("fp32"):  # the tiny layer's init: trunc_normal_(std) with the default bounds +-2
                torch.nn.init.trunc_normal_(t, mean=0.0, std=w["std"], generator=gen)
            else:
                t.normal_(0.0, w["std"], generator=gen)
            p.data = t.to(pdtype)
        bias = (torch.rand(e, generator=gen, device=device) * 2 - 1) * w["bias"]
        if w["zipf"]:
            # Zipf(s)-shaped per-expert boost over a random expert order, plus a
            # tail of 20 experts pushed below every score: the top expert gets
            # ~10x the mean load and those 20 experts get no tokens.
            ranks = torch.randperm(e, generator=gen, device=device).float() + 1.0
            bias = bias + 0.25 * ranks.pow(-w["zipf"]) - 1.0 * (ranks > e - 20).float()
        moe.expert_bias.copy_(bias)
        moe.tokens_per_expert.zero_()
    if w.get("fp8"):
        from torchtitan_amd.quantization import Float8GroupedMMConverter

        Float8GroupedMMConverter.Config(fqns=["experts"]).build(
            parallel_dims=_NO_PARALLEL, model_compile_enabled=False).convert(moe)
    if w.get("mxfp8"):
        from torchtitan_amd.quantization import MXFP8Converter

        MXFP8Converter.Config(fqns=["experts"]).build(
            parallel_dims=_NO_PARALLEL, model_compile_enabled=False).convert(moe)
    return moe


def cpu_model() -> str:
    """The host CPU's model name (as lscpu prints it), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(threads)
    return threads


def _time_reference_ops(params: dict, cfg, xs: torch.Tensor, gs: torch.Tensor, label: str) -> float:
    """Median of 3 forward + backward passes of the reference op sequence on the
    CPU after 1 warmup, in seconds."""
    from oracle import moe_ref as R

    times = []
    for it in range(4):
        for p in params.values():
            p.grad = None
        xi = xs.clone().requires_grad_(True)
        t0 = time.perf_counter()
        out = R.moe_forward_reference_ops(params, xi, cfg)
        out.backward(gs)
        times.append(time.perf_counter() - t0)
        print(f"[bench] cpu baseline {label} iteration {it}: {times[-1]:.3f} s", file=sys.stderr, flush=True)
    return statistics.median(times[1:])


def _router_cfg(w: dict):
    from oracle import moe_ref as R

    return R.RouterCfg(num_experts=w["experts"], top_k=w["top_k"], score_func=w["score_func"],
                       num_expert_groups=w["groups"], num_limited_groups=w["limited"],
                       route_norm=w["route_norm"], route_scale=w["route_scale"])


def cpu_baseline(moe, w: dict, x: torch.Tensor, g: torch.Tensor, n_tokens: int) -> dict:
    """The reference's CPU MoE path (oracle restatement of moe.py:380-477 with the
    same torch calls; histc -> bincount on the CPU) on the first n_tokens tokens,
    forward + backward, 1 warmup + median of 3, on this host's cores."""
    from oracle import moe_ref as R

    threads = _cpu_threads()
    sd = {k: v.detach().cpu() for k, v in moe.state_dict().items()}
    params = {"gate": sd["router.gate.weight"], "expert_bias": sd["expert_bias"]}
    if w.get("gptoss"):
        params["gate_bias"] = sd["router.gate.bias"]
        params.update({k: sd[f"experts.{k}"] for k in ("mlp1_weight", "mlp1_bias", "mlp2_weight", "mlp2_bias")})
    else:
        params.update(w1=sd["experts.w1"], w2=sd["experts.w2"], w3=sd["experts.w3"])
    if w["shared_hidden"]:
        params.update(sw1=sd["shared_experts.w1.weight"], sw2=sd["shared_experts.w2.weight"],
                      sw3=sd["shared_experts.w3.weight"])
    for k, p in params.items():
        if k != "expert_bias":
            p.requires_grad_(True)
    grouped = w.get("grouped", True)
    cfg = R.MoECfg(router=_router_cfg(w), dim=w["dim"], hidden_dim=w["hidden"],
                   score_before_experts=w["score_before"], use_grouped_mm=grouped,
                   has_shared=bool(w["shared_hidden"]), expert_kind="gptoss" if w.get("gptoss") else "swiglu")
    xs = x.reshape(-1, w["dim"])[:n_tokens].detach().cpu().reshape(1, n_tokens, w["dim"])
    gs = g.reshape(-1, w["dim"])[:n_tokens].detach().cpu().reshape(1, n_tokens, w["dim"])
    t = _time_reference_ops(params, cfg, xs, gs, w["desc"])
    print(f"[bench] cpu baseline: {n_tokens} tokens, {threads} threads, {t:.2f} s/iter", file=sys.stderr, flush=True)
    experts = "bf16 torch._grouped_mm experts" if grouped else f"{x.dtype} for-loop experts"
    return {
        "value": n_tokens * w["top_k"] / t,
        "unit": "routed tokens/s",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"reference op sequence (torch ops on the CPU, {experts}) fwd+bwd on "
                   f"{'all' if n_tokens == w['bs'] * w['slen'] else 'the first'} {n_tokens} of "
                   f"{w['bs'] * w['slen']} tokens of the same layer; median of 3 after 1 warmup; {t:.2f} s/iter"),
    }


def cpu_baseline_tiny(seed: int = 0) -> dict:
    """The tiny fp32 layer (dim 256, 8 experts, top-2 softmax, hidden 512, no
    shared expert, 4096 tokens) on the CPU through the reference op sequence in
    both expert modes: bf16 torch._grouped_mm (use_grouped_mm=True, the default)
    and the fp32 per-expert for-loop (moe.py:24-50). Inputs are drawn on the CPU
    from one seeded generator in the order gate, w1, w2, w3, bias, x, g."""
    from oracle import moe_ref as R

    w = WORKLOADS["c1"]
    threads = _cpu_threads()
    n, d, e, h = w["bs"] * w["slen"], w["dim"], w["experts"], w["hidden"]
    gen = torch.Generator().manual_seed(seed)

    def tn(*shape):
        return torch.nn.init.trunc_normal_(torch.empty(shape), mean=0.0, std=w["std"], generator=gen)

    params = {"gate": tn(e, d), "w1": tn(e, h, d), "w2": tn(e, d, h), "w3": tn(e, h, d), "expert_bias": torch.zeros(e)}
    x = torch.randn(1, n, d, generator=gen)
    g = torch.randn(1, n, d, generator=gen)
    for k, p in params.items():
        if k != "expert_bias":
            p.requires_grad_(True)
    out = {"cores": threads, "cpu_model": cpu_model(), "kind": "port", "unit": "routed tokens/s",
           "sample": f"all {n} tokens, fp32 parameters and activations; median of 3 after 1 warmup"}
    for grouped, key in ((True, "grouped_mm_bf16"), (False, "for_loop_fp32")):
        cfg = R.MoECfg(router=_router_cfg(w), dim=d, hidden_dim=h, score_before_experts=w["score_before"],
                       use_grouped_mm=grouped, has_shared=False)
        t = _time_reference_ops(params, cfg, x, g, f"tiny fp32 layer ({key})")
        out[key] = round(n * w["top_k"] / t, 1)
    return out


def _gemm_peak(name: str) -> float:
    if name.startswith(("moe_fp8_", "moe_mxfp8_")):
        return PEAK_FP8_TFLOPS
    if name.startswith("moe_grouped_gemm_f32_"):
        return PEAK_FP32_TFLOPS
    return PEAK_BF16_TFLOPS


TRAFFIC_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def measured_traffic(workload: str, entry: str) -> int | None:
    """HBM bytes per launch of `entry` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (profiles/hbm_traffic_<workload>.txt, already
    scaled by the copy-kernel calibration), or None when that workload was not profiled."""
    path = os.path.join(TRAFFIC_DIR, f"hbm_traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if parts and not line.startswith("#") and parts[0] == entry and len(parts) == 5:
                return int(parts[4])
    return None


def gemm_ceiling(w: dict, dev: torch.device, reps: int = 10) -> dict:
    """hipBLASLt (through torch.bmm / torch.mm, contiguous bf16 operands) on the
    uniform-batch equivalents of the six expert GEMMs of workload w: E batches of
    M = N*K/E rows each (every expert with the mean load, no ragged tail, no
    fused epilogue), and the same work as one dense GEMM. A reference for what
    the vendor library reaches on these shapes on this GPU; not part of the step."""
    n, d, e, k, h = w["bs"] * w["slen"], w["dim"], w["experts"], w["top_k"], w["hidden"]
    m = n * k // e
    shapes = {  # name: (batch, rows, contraction, columns)
        "gate_up": (e, m, d, 2 * h), "down": (e, m, h, d), "bwd_dgu": (e, m, d, h),
        "bwd_dx": (e, m, 2 * h, d), "bwd_dw13": (e, 2 * h, m, d), "bwd_dw2": (e, d, m, h),
        "dense_gate_up": (1, n * k, d, 2 * h),
    }
    gen = torch.Generator(device=dev).manual_seed(0)
    out = {}
    for name, (b, mm, kk, nn) in shapes.items():
        a = torch.randn(b, mm, kk, generator=gen, device=dev).bfloat16()
        bm = torch.randn(b, kk, nn, generator=gen, device=dev).bfloat16()
        fn = (lambda: torch.mm(a[0], bm[0])) if b == 1 else (lambda: torch.bmm(a, bm))
        for _ in range(3):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ts = []
        for _ in range(reps):
            ev[0].record()
            fn()
            ev[1].record()
            ev[1].synchronize()
            ts.append(ev[0].elapsed_time(ev[1]))
        ms = statistics.median(ts)
        tf = 2.0 * b * mm * kk * nn / (ms * 1e-3) / 1e12
        out[name] = {"shape": [b, mm, kk, nn], "ms": round(ms, 4), "tflops": round(tf, 1),
                     "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
        print(f"[bench] library GEMM {name} {b}x[{mm}x{kk}]x[{kk}x{nn}]: {ms:.4f} ms {tf:.1f} TFLOP/s",
              file=sys.stderr, flush=True)
        del a, bm
    return out


def mover_ceiling(w: dict, dev: torch.device, reps: int = 10) -> dict:
    """torch's own kernels on the movers' shapes of workload w (R = N*K routed rows of D
    bf16): a fill of R rows (writes only), a copy of R rows (read and write), the row
    gather x[token] of N rows into R (the unscored permute's traffic) and the sum over
    the K rows of each token of a token-major [N, K, D] array (the combine's reads and
    writes without its random gather). What plain streaming kernels reach for these
    read/write mixes on this GPU; not part of the step."""
    n, d, k = w["bs"] * w["slen"], w["dim"], w["top_k"]
    r = n * k
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(n, d, generator=gen, device=dev).bfloat16()
    big = torch.randn(r, d, generator=gen, device=dev).bfloat16()
    dst = torch.empty_like(big)
    tok = torch.randint(0, n, (r,), generator=gen, device=dev)
    row = 2 * d
    cases = {  # name: (fn, bytes read, bytes written)
        "fill": (lambda: dst.zero_(), 0, r * row),
        "copy": (lambda: dst.copy_(big), r * row, r * row),
        "gather_rows": (lambda: torch.index_select(x, 0, tok, out=dst), n * row, r * row),
        "sum_k_rows": (lambda: torch.sum(big.view(n, k, d), dim=1), r * row, n * row),
    }
    out = {}
    for name, (fn, rd, wr) in cases.items():
        for _ in range(3):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ts = []
        for _ in range(reps):
            ev[0].record()
            fn()
            ev[1].record()
            ev[1].synchronize()
            ts.append(ev[0].elapsed_time(ev[1]))
        ms = statistics.median(ts)
        gbs = (rd + wr) / (ms * 1e-3) / 1e9
        out[name] = {"read_bytes": rd, "write_bytes": wr, "ms": round(ms, 4), "gbs": round(gbs, 1),
                     "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4)}
        print(f"[bench] torch {name}: {ms:.4f} ms {gbs:.1f} GB/s", file=sys.stderr, flush=True)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="kimi", choices=sorted(WORKLOADS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="also time the vendor library on uniform-batch equivalents of the six expert GEMMs")
    ap.add_argument("--mover-ceiling", action="store_true",
                    help="also time torch's fill, copy, row gather and K-row sum on the movers' shapes")
    ap.add_argument("--cpu-tokens", type=int, default=None,
                    help="tokens in the CPU baseline sample (default: all for kimi, 1024 for dsv3, else 8192)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MoE layer runs with all experts resident on a single "
              "MI355X (no expert parallelism, no collectives); --gpus above 1 is not supported.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    from torchtitan_amd import _lib

    _lib.lib()  # fail loudly if the HIP library is missing
    w = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n = w["bs"] * w["slen"]
    k = w["top_k"]
    moe = make_layer(w, dev, args.seed)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 1)
    adtype = torch.float32 if w.get("fp32") else torch.bfloat16
    x = torch.randn(w["bs"], w["slen"], w["dim"], generator=gen, device=dev).to(adtype)
    g = torch.randn(w["bs"], w["slen"], w["dim"], generator=gen, device=dev).to(adtype)
    x.requires_grad_(True)
    params = list(moe.parameters())

    def step():
        for p in params:
            p.grad = None
        x.grad = None
        out = moe(x)
        out.backward(g)

    print(f"[bench] workload {args.workload}: warmup {args.warmup}", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    with torch.no_grad():
        counts = moe.router(x.detach().view(-1, w["dim"]), moe.expert_bias)[2].cpu()

    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps

    # per-kernel table: the same number of steps again, every C-ABI launch
    # bracketed by HIP events on its stream
    timer = _lib.KernelTimer()
    _lib.set_timer(timer)
    print(f"[bench] per-kernel timing over {args.steps} steps", file=sys.stderr, flush=True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    _lib.set_timer(None)

    durations = timer.durations_ms()
    launch_args = timer.launch_args()
    kernels = {}
    for name, ds in sorted(durations.items()):
        per_step = len(ds) / args.steps
        avg = sum(ds) / len(ds)
        bound, work = kernel_work(name, w)
        if work is None:
            lb = [launch_bytes(name, a) for a in launch_args[name]]
            if all(v is not None for v in lb):
                work = sum(lb) / len(lb)  # bytes of the average launch, over the average launch time
        if bound == "mfma":
            peak = _gemm_peak(name)
            achieved, unit = work / (avg * 1e-3) / 1e12, "TFLOP/s"
        elif work is not None:
            achieved, peak, unit = work / (avg * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
        else:
            achieved, peak, unit = None, None, "GB/s"
        kernels[name] = {
            "launches_per_step": per_step, "avg_ms": round(avg, 4), "bound": bound,
            "achieved": round(achieved, 1) if achieved is not None else None, "unit": unit,
            "frac": round(achieved / peak, 4) if achieved is not None else None,
        }
    gemm_ms = sum(kernels[nm]["avg_ms"] * kernels[nm]["launches_per_step"] for nm in GEMM_ENTRIES if nm in kernels)
    gemm_flops = 18.0 * n * k * w["dim"] * w["hidden"]
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0
    dom = max(kernels, key=lambda nm: kernels[nm]["avg_ms"] * kernels[nm]["launches_per_step"])
    dk = kernels[dom]
    gemm_peak = (PEAK_FP8_TFLOPS if (w.get("fp8") or w.get("mxfp8")) else
                 PEAK_FP32_TFLOPS if (w.get("fp32") and not w.get("grouped", True)) else PEAK_BF16_TFLOPS)
    roofline = {
        "kernel": dom,
        "bound": dk["bound"],
        "achieved": dk["achieved"],
        "peak": _gemm_peak(dom) if dk["bound"] == "mfma" else PEAK_HBM_GBS,
        "unit": dk["unit"],
        "frac": dk["frac"],
        "traffic": measured_traffic(args.workload, dom),
        "traffic_source": (f"profiles/hbm_traffic_{args.workload}.txt: rocprofv3 FETCH_SIZE and WRITE_SIZE per "
                           f"dispatch of the committed build, scaled by a copy-kernel calibration; not measured "
                           f"in this run"),
    }
    mover = ("moe_permute", "moe_combine", "moe_combine_bwd", "moe_permute_bwd")
    mover_ms = sum(kernels[m]["avg_ms"] for m in mover if m in kernels)
    mover_bytes = sum(kernel_work(m, w)[1] for m in mover if m in kernels)

    cpu = cpu_tiny = None
    if not args.no_cpu_baseline:
        cpu_tokens = args.cpu_tokens or {"dsv3": 1024, "kimi": n}.get(args.workload, 8192)
        cpu = cpu_baseline(moe, w, x, g, min(cpu_tokens, n))
        if args.workload == "kimi":
            cpu_tiny = cpu_baseline_tiny()

    line = {
        "metric": "MoE layer fwd+bwd routed tokens/s; grouped-GEMM TFLOPS as % of MFMA peak",
        "value": round(n * k / (ms * 1e-3), 1),
        "unit": "routed tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp8 e4m3 (grouped GEMMs), bf16 elsewhere" if w.get("fp8") else
                  "fp32" if (w.get("fp32") and not w.get("grouped", True)) else
                  "fp32 (bf16 grouped GEMMs)" if w.get("fp32") else
                  "MXFP8 e4m3 + e8m0 block-32 scales (grouped GEMMs), bf16 elsewhere" if w.get("mxfp8") else "bf16"),
        "data": "synthetic (random-init weights, x ~ N(0,1), g ~ N(0,1))",
        "config": {
            "workload": f"{w['desc']}: N={n} tokens (bs {w['bs']} x seq {w['slen']}), dim {w['dim']}, "
                        f"{w['experts']} experts top-{k} {w['score_func']}"
                        f"{' group-limited ' + str(w['limited']) + '/' + str(w['groups']) if w['groups'] else ''}"
                        f" + bias, hidden {w['hidden']}, shared hidden {w['shared_hidden']}, fwd+bwd",
            "tokens": n, "dim": w["dim"], "num_experts": w["experts"], "top_k": k,
            "hidden": w["hidden"], "shared_hidden": w["shared_hidden"],
            "parallelism": "single GPU, all experts resident",
        },
        "tokens_per_s": round(n / (ms * 1e-3), 1),
        "grouped_gemm": {
            "ms_per_step": round(gemm_ms, 4),
            "tflops": round(gemm_tflops, 1),
            "frac_of_peak": round(gemm_tflops / gemm_peak, 4),
        },
        "permute_combine": {
            "ms_per_step": round(mover_ms, 4),
            "gbs": round(mover_bytes / (mover_ms * 1e-3) / 1e9, 1) if mover_ms else None,
            "frac_of_peak": round(mover_bytes / (mover_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if mover_ms else None,
        },
        "expert_load": {"max": int(counts.max()), "mean": float(counts.float().mean()),
                        "empty": int((counts == 0).sum())},
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_tiny_fp32_layer": cpu_tiny,
    }
    if args.gemm_ceiling:
        line["library_gemm_uniform_batch"] = gemm_ceiling(w, dev)
    if args.mover_ceiling:
        line["torch_streaming_kernels"] = mover_ceiling(w, dev)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
