"""bench.py's algorithmic work per launch, derived here a second way: from the list of
tensors each kernel reads and writes (shape and element size), not from the closed
forms in bench.kernel_work. Runs on the CPU (no kernel is launched)."""

import subprocess
import sys

import pytest

import bench


def _tensors(wl):
    w = bench.WORKLOADS[wl]
    n, d, k, h = w["bs"] * w["slen"], w["dim"], w["top_k"], w["hidden"]
    r = n * k
    row = 4 if w.get("fp32") else 2
    t = {  # name: bytes
        "x": n * d * row, "routed": r * d * row, "out": n * d * row, "shared_out": n * d * row,
        "grad_out": n * d * row, "grad_routed": r * d * row, "grad_x": n * d * row,
        "slot_pos": n * k * 4, "tok_pos": n * k * 4, "scores_sorted": r * 4, "grad_scores_sorted": r * 4,
    }
    return w, t, (n, d, k, h, r)


def _movers(wl):
    w, t, _ = _tensors(wl)
    sb = w["score_before"]
    return {
        "moe_permute": [t["x"], t["routed"], t["slot_pos"]] + ([t["scores_sorted"]] if sb else []),
        "moe_combine": [t["routed"], t["shared_out"], t["out"], t["tok_pos"]] + ([] if sb else [t["scores_sorted"]]),
        "moe_combine_bwd": ([t["grad_out"], t["grad_routed"], t["slot_pos"]] if sb else
                            [t["grad_out"], t["routed"], t["grad_routed"], t["tok_pos"], t["scores_sorted"],
                             t["grad_scores_sorted"]]),
        "moe_permute_bwd": ([t["grad_routed"], t["x"], t["grad_x"], t["tok_pos"], t["scores_sorted"],
                             t["grad_scores_sorted"]] if sb else [t["grad_routed"], t["grad_x"], t["tok_pos"]]),
    }


@pytest.mark.parametrize("wl", ["kimi", "dsv3", "gptoss_20b", "c1", "c1_grouped", "zipf"])
def test_mover_bytes_follow_the_score_placement_and_row_type(wl):
    w = bench.WORKLOADS[wl]
    for name, parts in _movers(wl).items():
        bound, nbytes = bench.kernel_work(name, w)
        assert bound == "hbm"
        assert nbytes == sum(parts), (wl, name, nbytes, sum(parts))


@pytest.mark.parametrize("wl", ["kimi", "dsv3", "kimi_fp8"])
def test_gemm_flops_are_two_per_multiply_add(wl):
    w, _, (n, d, k, h, r) = _tensors(wl)
    # (rows, contraction, columns) of each product, summed over the experts
    shapes = {"gate_up": (r, d, 2 * h), "down": (r, h, d), "bwd_dgu": (r, d, h), "bwd_dx": (r, 2 * h, d),
              "bwd_dw13": (2 * h, r, d), "bwd_dw2": (d, r, h)}
    prefix = "moe_fp8_gemm_" if w.get("fp8") else "moe_grouped_gemm_"
    for mode, (m, kk, nn) in shapes.items():
        assert bench.kernel_work(prefix + mode, w) == ("mfma", float(2 * m * kk * nn))


def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True, timeout=300)
    assert res.returncode != 0
    assert "one GPU" in (res.stdout + res.stderr) or "1 GPU" in (res.stdout + res.stderr)
