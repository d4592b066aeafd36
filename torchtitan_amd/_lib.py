"""ctypes binding of libmoe_mi355x.so (declared in include/moe_mi355x.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (same soname, libamdhip64.so.7). There is no
fallback: if the library is missing, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmoe_mi355x.so")
_lib = None
_lock = threading.Lock()

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float

# name -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "moe_router_fwd": [P, P, I64, I32, I32, I32, I32, I32, I32, F32, I32, P, P, P, P],
    "moe_router_bwd": [P, P, P, I64, I32, I32, I32, I32, F32, P, P],
    "moe_gate_grad_split3": [P, I64, I32, P, P],
    "moe_gate_dw_reduce": [P, I32, I32, I32, P, P],
    "moe_swiglu_fwd": [P, P, I64, I32, I32, P, P],
    "moe_swiglu_bwd": [P, P, P, I64, I32, I32, P, P],
    "moe_reorder_workspace_bytes": [I64, I32],
    "moe_histogram": [P, I64, I32, I32, P, I64, P, P, P],
    "moe_reorder": [P, P, I64, I32, I32, P, I64, P, P, P, P, P, P, P],
    "moe_reorder_noalloc": [P, P, I64, I32, I32, P, P, P, P, P, P, P],
    "moe_reorder_bwd": [P, P, I64, I32, P, P],
    "moe_permute": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_permute_bwd": [P, P, P, P, I64, I32, I32, I32, I32, P, P, P],
    "moe_combine": [P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_combine_bwd": [P, P, P, P, P, I64, I32, I32, I32, P, P, P],
    "moe_grouped_swiglu_fwd": [P, P, P, P, P, I64, I32, I32, I32, P, P, P, P, P],
    "moe_grouped_swiglu_bwd": [P, P, P, P, P, P, P, P, P, I64, I32, I32, I32, P, P, P, P, P, P],
    "moe_grouped_gemm_gate_up": [P, P, P, P, I64, I32, I32, I32, P, P, P, P],
    "moe_grouped_gemm_down": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_bwd_dgu": [P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_bwd_dx": [P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_bwd_dw13": [P, P, P, I64, I32, I32, I32, P, P, P],
    "moe_grouped_gemm_bwd_dw2": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_swiglu_pointwise_f32": [P, P, P, I64, P],
    "moe_grouped_gemm_f32_gate_up": [P, P, P, P, I64, I32, I32, I32, P, P, P, P],
    "moe_grouped_gemm_f32_down": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_f32_bwd_dgu": [P, P, P, P, P, I64, I32, I32, I32, P, P, P],
    "moe_grouped_gemm_f32_bwd_dx": [P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_f32_bwd_dw": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_fp8_padded_rows": [I64, I32],
    "moe_fp8_quant_rows": [P, I64, I32, P, P, P],
    "moe_fp8_quant_cols_t": [P, I32, I32, I32, P, I64, I64, P, I64, P],
    "moe_fp8_quant_cols_t_amax": [P, P, I32, I32, I32, P, I64, I64, P, I64, P],
    "moe_fp8_quant_rows_colamax": [P, I32, I32, I32, P, P, P, P],
    "moe_fp8_quant_tokens_t": [P, P, I64, I32, I32, I64, P, P, P],
    "moe_fp8_quant_tokens_t_amax": [P, P, P, I64, I32, I32, I64, P, P, P],
    "moe_fp8_quant_rows_groupamax": [P, P, I64, I32, I32, I32, P, P, P, P],
    "moe_fp8_quant_rows_groupamax_gather": [P, I64, P, P, P, I64, I32, I32, P, P, P, P],
    "moe_fp8_quant_tokens_t_amax_gather": [P, I64, P, P, P, P, I64, I32, I32, I64, P, P, P],
    "moe_fp8_gemm_gate_up": [P, P, P, P, P, P, P, I64, I32, I32, I32, P, P, P, P],
    "moe_fp8_gemm_down": [P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_fp8_gemm_bwd_dgu": [P, P, P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_fp8_gemm_bwd_dx": [P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_fp8_gemm_bwd_dw13": [P, P, P, P, P, I64, I64, I32, I32, I32, P, P, P],
    "moe_fp8_gemm_bwd_dw2": [P, P, P, P, P, I64, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_oss_gate_up": [P, P, P, P, I64, I32, I32, I32, F32, P, P, P, P],
    "moe_grouped_gemm_oss_down": [P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_oss_bwd_dgu": [P, P, P, P, P, I64, I32, I32, I32, F32, P, P],
    "moe_grouped_gemm_oss_bwd_dx": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_gemm_oss_bwd_dw1": [P, P, P, I64, I32, I32, I32, P, P],
    "moe_grouped_col_sum": [P, I64, P, I64, I32, I32, P, I64, I32, P],
    "moe_mxfp8_padded_rows": [I64, I32],
    "moe_mxfp8_quant_rows": [P, I64, I32, P, P, P],
    "moe_mxfp8_quant_cols_t": [P, I32, I32, I32, P, I64, I64, P, I64, I64, P],
    "moe_mxfp8_quant_tokens_t": [P, P, I64, I32, I32, I64, P, P, P],
    "moe_mxfp8_quant_dual_cols": [P, I32, I32, I32, P, P, P, I64, I64, P, I64, I64, P],
    "moe_mxfp8_quant_dual_tokens": [P, P, I64, I32, I32, I64, P, P, P, P, P],
    "moe_mxfp8_quant_dual_tokens_gather": [P, I64, P, P, P, I64, I32, I32, I64, P, P, P, P, P],
    "moe_mxfp8_gemm_gate_up": [P, P, P, P, P, P, P, I64, I32, I32, I32, P, P, P, P],
    "moe_mxfp8_gemm_down": [P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_mxfp8_gemm_bwd_dgu": [P, P, P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_mxfp8_gemm_bwd_dx": [P, P, P, P, P, I64, I32, I32, I32, P, P],
    "moe_mxfp8_gemm_bwd_dw13": [P, P, P, P, P, I64, I64, I32, I32, I32, P, P, P],
    "moe_mxfp8_gemm_bwd_dw2": [P, P, P, P, P, I64, I64, I32, I32, I32, P, P],
    "moe_expert_bias_update": [P, P, P, P, I32, I32, P],
    "moe_ep_permute_indices": [P, I32, I32, I64, P, P, P],
    "moe_ep_permute_pad_indices": [P, I32, I32, I32, I64, P, P, P, P],
    "moe_gather_rows": [P, I64, P, I64, I32, I32, P, P],
    "moe_scatter_rows": [P, P, I64, I32, I32, P, I64, P],
}
_RESTYPES = {"moe_reorder_workspace_bytes": ctypes.c_int64, "moe_fp8_padded_rows": ctypes.c_int64,
             "moe_mxfp8_padded_rows": ctypes.c_int64}

_ERRORS = {
    -1: "invalid argument",
    -2: "unsupported shape",
    -3: "kernel launch failed",
    -4: "workspace too small",
}


class MoEKernelError(RuntimeError):
    pass


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise MoEKernelError(
                    f"{_LIB_PATH} is missing: build the MI355X kernels first "
                    "(python -m torchtitan_amd.build)"
                )
            handle = ctypes.CDLL(_LIB_PATH)
            for name, argtypes in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        raise MoEKernelError(f"{what}: {_ERRORS.get(status, 'error')} (status {status})")


class KernelTimer:
    """Brackets every C-ABI launch with HIP events on the stream it is enqueued
    on (torch's current stream), keyed by entry-point name. Events are only
    read after the caller synchronises (``durations_ms``)."""

    def __init__(self) -> None:
        self.events: dict[str, list] = {}

    def durations_ms(self) -> dict[str, list[float]]:
        return {k: [a.elapsed_time(b) for a, b, _ in v] for k, v in self.events.items()}

    def launch_args(self) -> dict[str, list[tuple]]:
        """The C-ABI arguments of every timed launch (ints and pointers), in order."""
        return {k: [args for _, _, args in v] for k, v in self.events.items()}


_timer: KernelTimer | None = None


def set_timer(timer: KernelTimer | None) -> None:
    global _timer
    _timer = timer


def call(name: str, *args) -> None:
    """Calls entry point `name` and raises on a non-zero status. When a
    KernelTimer is installed, the launch is bracketed by events."""
    fn = getattr(lib(), name)
    t = _timer
    if t is None:
        check(fn(*args), name)
        return
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    st = fn(*args)
    b.record()
    check(st, name)
    t.events.setdefault(name, []).append((a, b, args))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise MoEKernelError(
                "the MI355X MoE kernels run on the GPU only; got a tensor on " f"{t.device}"
            )
