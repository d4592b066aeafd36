// Elementwise kernels around two dense GEMM blocks of the MoE layer:
//
//  * the router gate's backward (the fp32 autocast gate of
//    torchtitan/models/common/moe.py:229-232): the fp32 logit gradient is split
//    exactly into three bf16 terms so that dx and dW run as bf16 GEMMs with fp32
//    accumulation (products exact in fp32), and the dW partial sums are reduced
//    and rounded once;
//  * the shared expert's SwiGLU (torchtitan/models/common/feed_forward.py:53-54,
//    w2(silu(w1 x) * w3 x)) forward and its autograd, between the library GEMMs.
//
// Each replaces a chain of torch elementwise launches (8 for the split, 4 for the
// reduction, 2 and 3 for the SwiGLU) by one pass over HBM, with the same fp32
// operations in the same order and the same roundings, so the results are the
// torch op sequence's bits.
#include "common.h"

namespace moe {

// ---------------------------------------------------------------------------
// gate backward: d [N, C] fp32 -> [N, 3C] bf16 (hi | mid | lo), hi + mid + lo == d
// ---------------------------------------------------------------------------
// hi = bf16(d), mid = bf16(d - hi), lo = bf16((d - hi) - mid): each subtraction is
// exact in fp32 (a value minus its own rounding to fewer bits), so the three terms
// carry d's 24 significand bits 8 at a time.
__global__ __launch_bounds__(256) void grad_split3_kernel(const float* __restrict__ d, int64_t n_rows, int C,
                                                          uint16_t* __restrict__ out) {
  const int cq = C / 4;
  const int64_t total = n_rows * cq;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cq;
    const int c = (int)(i - r * cq) * 4;
    const float4 v = *(const float4*)(d + r * C + c);
    const float f[4] = {v.x, v.y, v.z, v.w};
    float hi[4], mid[4], lo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      hi[q] = round_bf(f[q]);
      const float rem = f[q] - hi[q];
      mid[q] = round_bf(rem);
      lo[q] = round_bf(rem - mid[q]);
    }
    uint16_t* o = out + r * (3 * (int64_t)C) + c;
    *(uint2*)o = pack4(hi);
    *(uint2*)(o + C) = pack4(mid);
    *(uint2*)(o + 2 * C) = pack4(lo);
  }
}

// partials [P, 3E, D] fp32 (P = 1 or 2 token halves) -> dW [E, D] bf16:
// t = p0 (+ p1) for each of the hi, mid, lo row blocks, dW = bf16((t_hi + t_mid) + t_lo)
template <int P>
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ part, int64_t ed,
                                                        uint16_t* __restrict__ out) {
  const int64_t total = ed / 4;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t o = i * 4;
    float t[3][4];
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const float4 a = *(const float4*)(part + b * ed + o);
      t[b][0] = a.x; t[b][1] = a.y; t[b][2] = a.z; t[b][3] = a.w;
      if constexpr (P == 2) {
        const float4 c = *(const float4*)(part + 3 * ed + b * ed + o);
        t[b][0] = t[b][0] + c.x; t[b][1] = t[b][1] + c.y; t[b][2] = t[b][2] + c.z; t[b][3] = t[b][3] + c.w;
      }
    }
    float s[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) s[q] = (t[0][q] + t[1][q]) + t[2][q];
    *(uint2*)(out + o) = pack4(s);
  }
}

// ---------------------------------------------------------------------------
// shared expert SwiGLU
// ---------------------------------------------------------------------------
// torch's GPU formulas in the op math type: silu(x) = x / (1 + exp(-x)),
// silu_backward(dy, x) = dy * sigmoid * (1 + x * (1 - sigmoid)) with
// sigmoid = 1 / (1 + exp(-x)); the exponential is computed once for both. For bf16
// the vector kernels divide in the reciprocal form of the grouped GEMMs' epilogues
// (silu_sig in common.h: IEEE division's results for every bf16 input) where a
// chunk's values lie in its range in every lane.

// the range of a chunk's V values, for silu_fast_wave
template <int V>
__device__ __forceinline__ bool chunk_fast(const float (&g)[V]) {
  float lo = g[0], hi = g[0];
#pragma unroll
  for (int q = 1; q < V; ++q) {
    lo = fminf(lo, g[q]);
    hi = fmaxf(hi, g[q]);
  }
  return silu_fast_wave(lo, hi);
}

// h = rnd(rnd(silu(a1)) * a3), T = bf16 (rnd = round to bf16) or fp32 (rnd = identity)
template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(const T* __restrict__ a1, const T* __restrict__ a3,
                                                         int64_t n, T* __restrict__ h) {
  constexpr int V = Chunk<T>::kN;
  const int64_t nv = n / V;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * blockDim.x) {
    float g[V], u[V], o[V];
    Chunk<T>::unpack(*(const uint4*)(a1 + i * V), g);
    Chunk<T>::unpack(*(const uint4*)(a3 + i * V), u);
    float d[V];
#pragma unroll
    for (int q = 0; q < V; ++q) d[q] = silu_den(g[q]);
    if (sizeof(T) == 2 && chunk_fast<V>(g)) {
#pragma unroll
      for (int q = 0; q < V; ++q) o[q] = Chunk<T>::round(silu_sig<true>(g[q], d[q]).silu) * u[q];
    } else {
#pragma unroll
      for (int q = 0; q < V; ++q) o[q] = Chunk<T>::round(silu_sig<false>(g[q], d[q]).silu) * u[q];
    }
    *(uint4*)(h + i * V) = Chunk<T>::pack(o);
  }
}

// dgu [rows, 2 Hs]: dg = rnd(silu_backward(rnd(dh * a3), a1)) in columns [0, Hs),
// du = rnd(dh * rnd(silu(a1))) in [Hs, 2 Hs); dh, a1, a3 [rows, Hs]
template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const T* __restrict__ dh, const T* __restrict__ a1,
                                                         const T* __restrict__ a3, int64_t rows, int hs,
                                                         T* __restrict__ dgu) {
  constexpr int V = Chunk<T>::kN;
  const int cv = hs / V;
  const int64_t nv = rows * cv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cv;
    const int c = (int)(i - r * cv) * V;
    const int64_t off = r * hs + c;
    float d[V], g[V], u[V], dg[V], du[V];
    Chunk<T>::unpack(*(const uint4*)(dh + off), d);
    Chunk<T>::unpack(*(const uint4*)(a1 + off), g);
    Chunk<T>::unpack(*(const uint4*)(a3 + off), u);
    float den[V];
    SiluSig f[V];
#pragma unroll
    for (int q = 0; q < V; ++q) den[q] = silu_den(g[q]);
    if (sizeof(T) == 2 && chunk_fast<V>(g)) {
#pragma unroll
      for (int q = 0; q < V; ++q) f[q] = silu_sig<true>(g[q], den[q]);
    } else {
#pragma unroll
      for (int q = 0; q < V; ++q) f[q] = silu_sig<false>(g[q], den[q]);
    }
#pragma unroll
    for (int q = 0; q < V; ++q) {
      const float s = Chunk<T>::round(f[q].silu);
      const float sg = f[q].sig;
      const float dsl = Chunk<T>::round(d[q] * u[q]);
      du[q] = d[q] * s;
      dg[q] = dsl * sg * (1.0f + g[q] * (1.0f - sg));
    }
    T* o = dgu + r * (2 * (int64_t)hs) + c;
    *(uint4*)o = Chunk<T>::pack(dg);
    *(uint4*)(o + hs) = Chunk<T>::pack(du);
  }
}

// widths that are not a multiple of the 16-byte chunk: one element per thread
template <typename T>
__device__ __forceinline__ float ld1(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 2) return bf2f(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}
template <typename T>
__device__ __forceinline__ void st1(T* p, int64_t i, float v) {
  if constexpr (sizeof(T) == 2) ((uint16_t*)p)[i] = (uint16_t)f2bf(v);
  else ((float*)p)[i] = v;
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_fwd_scalar_kernel(const T* __restrict__ a1, const T* __restrict__ a3,
                                                                int64_t n, T* __restrict__ h) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float g = ld1(a1, i);
    st1(h, i, Chunk<T>::round(g / (1.0f + expf(-g))) * ld1(a3, i));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void swiglu_bwd_scalar_kernel(const T* __restrict__ dh, const T* __restrict__ a1,
                                                                const T* __restrict__ a3, int64_t rows, int hs,
                                                                T* __restrict__ dgu) {
  const int64_t n = rows * hs;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / hs;
    const int c = (int)(i - r * hs);
    const float d = ld1(dh, i), g = ld1(a1, i), u = ld1(a3, i);
    const float e = expf(-g);
    const float s = Chunk<T>::round(g / (1.0f + e));
    const float sg = 1.0f / (1.0f + e);
    const float dsl = Chunk<T>::round(d * u);
    st1(dgu, r * (2 * (int64_t)hs) + c, dsl * sg * (1.0f + g * (1.0f - sg)));
    st1(dgu, r * (2 * (int64_t)hs) + hs + c, d * s);
  }
}

static bool aligned16(const void* a, const void* b, const void* c, const void* d = nullptr) {
  return (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)d) & 15) == 0;
}

static int elementwise_grid(int64_t work) {
  int64_t g = (work + 255) / 256;
  if (g > 8192) g = 8192;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace moe

using namespace moe;

MOE_API int moe_gate_grad_split3(const float* grad_logits, int64_t n_rows, int32_t n_cols, uint16_t* terms,
                                 hipStream_t stream) {
  if (n_rows < 0 || n_cols <= 0 || n_cols % 4 != 0) return kErrUnsupportedShape;
  if (n_rows == 0) return kOk;
  if (!grad_logits || !terms || !aligned16(grad_logits, terms, nullptr)) return kErrInvalidArgument;
  const int64_t work = n_rows * (n_cols / 4);
  hipLaunchKernelGGL(grad_split3_kernel, dim3(elementwise_grid(work)), dim3(256), 0, stream, grad_logits, n_rows,
                     (int)n_cols, terms);
  return launch_status();
}

MOE_API int moe_gate_dw_reduce(const float* partials, int32_t n_parts, int32_t n_experts, int32_t dim,
                               uint16_t* grad_weight, hipStream_t stream) {
  if (n_parts != 1 && n_parts != 2) return kErrInvalidArgument;
  if (n_experts <= 0 || dim <= 0 || dim % 4 != 0) return kErrUnsupportedShape;
  if (!partials || !grad_weight || !aligned16(partials, grad_weight, nullptr)) return kErrInvalidArgument;
  const int64_t ed = (int64_t)n_experts * dim;
  const dim3 grid(elementwise_grid(ed / 4)), block(256);
  if (n_parts == 2)
    hipLaunchKernelGGL(dw_reduce_kernel<2>, grid, block, 0, stream, partials, ed, grad_weight);
  else
    hipLaunchKernelGGL(dw_reduce_kernel<1>, grid, block, 0, stream, partials, ed, grad_weight);
  return launch_status();
}

MOE_API int moe_swiglu_fwd(const void* a1, const void* a3, int64_t n_rows, int32_t hidden, int32_t dtype, void* h,
                           hipStream_t stream) {
  if (dtype != MOE_DTYPE_BF16 && dtype != MOE_DTYPE_FP32) return kErrInvalidArgument;
  const int v = dtype == MOE_DTYPE_BF16 ? 8 : 4;
  if (n_rows < 0 || hidden <= 0) return kErrUnsupportedShape;
  if (n_rows == 0) return kOk;
  if (!a1 || !a3 || !h) return kErrInvalidArgument;
  const int64_t n = n_rows * hidden;
  if (hidden % v != 0 || !aligned16(a1, a3, h)) {
    const dim3 grid1(elementwise_grid(n)), block1(256);
    if (dtype == MOE_DTYPE_BF16)
      hipLaunchKernelGGL(swiglu_fwd_scalar_kernel<uint16_t>, grid1, block1, 0, stream, (const uint16_t*)a1,
                         (const uint16_t*)a3, n, (uint16_t*)h);
    else
      hipLaunchKernelGGL(swiglu_fwd_scalar_kernel<float>, grid1, block1, 0, stream, (const float*)a1,
                         (const float*)a3, n, (float*)h);
    return launch_status();
  }
  const dim3 grid(elementwise_grid(n / v)), block(256);
  if (dtype == MOE_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_fwd_kernel<uint16_t>, grid, block, 0, stream, (const uint16_t*)a1,
                       (const uint16_t*)a3, n, (uint16_t*)h);
  else
    hipLaunchKernelGGL(swiglu_fwd_kernel<float>, grid, block, 0, stream, (const float*)a1, (const float*)a3, n,
                       (float*)h);
  return launch_status();
}

MOE_API int moe_swiglu_bwd(const void* dh, const void* a1, const void* a3, int64_t n_rows, int32_t hidden,
                           int32_t dtype, void* dgu, hipStream_t stream) {
  if (dtype != MOE_DTYPE_BF16 && dtype != MOE_DTYPE_FP32) return kErrInvalidArgument;
  const int v = dtype == MOE_DTYPE_BF16 ? 8 : 4;
  if (n_rows < 0 || hidden <= 0) return kErrUnsupportedShape;
  if (n_rows == 0) return kOk;
  if (!dh || !a1 || !a3 || !dgu) return kErrInvalidArgument;
  if (hidden % v != 0 || !aligned16(dh, a1, a3, dgu)) {
    const dim3 grid1(elementwise_grid(n_rows * hidden)), block1(256);
    if (dtype == MOE_DTYPE_BF16)
      hipLaunchKernelGGL(swiglu_bwd_scalar_kernel<uint16_t>, grid1, block1, 0, stream, (const uint16_t*)dh,
                         (const uint16_t*)a1, (const uint16_t*)a3, n_rows, (int)hidden, (uint16_t*)dgu);
    else
      hipLaunchKernelGGL(swiglu_bwd_scalar_kernel<float>, grid1, block1, 0, stream, (const float*)dh,
                         (const float*)a1, (const float*)a3, n_rows, (int)hidden, (float*)dgu);
    return launch_status();
  }
  const dim3 grid(elementwise_grid(n_rows * (hidden / v))), block(256);
  if (dtype == MOE_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_bwd_kernel<uint16_t>, grid, block, 0, stream, (const uint16_t*)dh,
                       (const uint16_t*)a1, (const uint16_t*)a3, n_rows, (int)hidden, (uint16_t*)dgu);
  else
    hipLaunchKernelGGL(swiglu_bwd_kernel<float>, grid, block, 0, stream, (const float*)dh, (const float*)a1,
                       (const float*)a3, n_rows, (int)hidden, (float*)dgu);
  return launch_status();
}
