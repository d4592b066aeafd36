// Shared device helpers for the MI355X (gfx950) MoE kernels.
//
// Everything here is written for CDNA4: 64-wide wavefronts, LDS-resident
// scratch, bf16 stored as raw uint16_t and widened to fp32 for arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_mi355x.h"

#define MOE_API extern "C" __attribute__((visibility("default")))

namespace moe {

constexpr int kWave = 64;

// Status codes returned by every C-ABI entry point (mirrored in include/moe_mi355x.h).
enum Status : int {
  kOk = 0,
  kErrInvalidArgument = -1,
  kErrUnsupportedShape = -2,
  kErrLaunch = -3,
  kErrWorkspace = -4,
};

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// ---------------------------------------------------------------------------
// bf16 <-> fp32. The narrowing conversion is round-to-nearest-even with NaN
// mapped to the canonical quiet NaN 0x7FC0, which is what torch's bf16 casts do.
// It runs on gfx950's v_cvt_pk_bf16_f32 (what clang emits for a float -> __bf16
// conversion) after NaNs are replaced by the canonical one; checked on the GPU
// against the integer formulation (u + 0x7fff + ((u >> 16) & 1)) >> 16, NaN ->
// 0x7fc0, for every fp32 bit pattern, alone and packed in pairs.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }

__device__ __forceinline__ float nan_canon(float f) { return f != f ? __uint_as_float(0x7fc00000u) : f; }

__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)nan_canon(f));
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// lo/hi bf16 of a packed dword
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const f32x2_t v = {nan_canon(lo), nan_canon(hi)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// silu(g) = g / d and sigmoid(g) = 1 / d with d = 1 + exp(-g), the quotients rounded
// as IEEE division rounds them (torch's kernels divide), without the general
// division's scaling and fix-up steps: the hardware reciprocal estimate refined by one
// Newton step on fused multiply-adds, then the quotient corrected once by its exact
// fused residual (Markstein, IBM J. Res. Dev. 34(1), 1990). For g in [-80, 3.38e38]
// d lies in [1, 2^116] and nothing over- or underflows; the results equal IEEE
// division there for every bf16 g (a GPU test compares all 65536 of them with
// torch's silu and sigmoid, -0 included), and a NaN g gives NaN either way. A piece of values
// with any g below -80 or above 3.38e38 in any lane takes the division (kFast false).
struct SiluSig { float silu, sig; };
__device__ __forceinline__ bool silu_fast_range(float g_min, float g_max) {
  return g_min >= -80.0f && g_max <= 3.38e38f;  // fminf / fmaxf drop NaN
}
// the same for every active lane of the wave, so that the choice is a scalar branch
// between two straight paths rather than both paths under lane masks
__device__ __forceinline__ bool silu_fast_wave(float g_min, float g_max) {
  return __builtin_expect(__builtin_amdgcn_ballot_w64(!silu_fast_range(g_min, g_max)) == 0, 1);
}
__device__ __forceinline__ float silu_den(float g) { return 1.0f + expf(-g); }
template <bool kFast>
__device__ __forceinline__ SiluSig silu_sig(float g, float d) {
  if constexpr (kFast) {
    float y = __builtin_amdgcn_rcpf(d);
    y = fmaf(fmaf(-d, y, 1.0f), y, y);
    const float q = g * y;
    // the quotient has g's sign (d > 0); the correction alone would turn -0 into +0
    return {copysignf(fmaf(fmaf(-d, q, g), y, q), g), y};
  } else {
    return {g / d, 1.0f / d};
  }
}

// Epilogue stores in 64-byte row pieces. An accumulator tile leaves lane (r, g),
// r = lane % 16, g = lane / 16, with 4 consecutive columns 4g .. 4g + 3 of row r
// in each 16-column block; for two adjacent blocks (lo, hi) packed to bf16, this
// returns the 8 columns 8g .. 8g + 7 of the 32-column span [lo | hi] of row r,
// gathered from the lanes of the same row, so that the four lanes of a row store
// 64 contiguous bytes with one 16-byte store each (instead of 32 bytes per block).
// The exchange is two lane-half swaps and two lane-row swaps of gfx950 (no LDS):
// with lo(g), hi(g) the pairs of lane row g (16 lanes), swapping the upper 32 lanes
// of lo with the lower 32 of hi gives [lo0 lo1 hi0 hi1] / [lo2 lo3 hi2 hi3], and
// swapping the odd rows of the first with the even rows of the second gives
// [lo0 lo2 hi0 hi2] / [lo1 lo3 hi1 hi3]: lane (r, g)'s columns 8g .. 8g + 3 and
// 8g + 4 .. 8g + 7. Data moves only between the lanes of one row r, which share
// their active state wherever the epilogues skip rows. (Cross-lane reads through
// the LDS crossbar cost bank-conflict cycles in every epilogue.)
__device__ __forceinline__ uint4 span64(uint2 lo, uint2 hi, int lane) {
  (void)lane;
  const auto x32 = __builtin_amdgcn_permlane32_swap(lo.x, hi.x, false, false);
  const auto y32 = __builtin_amdgcn_permlane32_swap(lo.y, hi.y, false, false);
  const auto x16 = __builtin_amdgcn_permlane16_swap(x32[0], x32[1], false, false);
  const auto y16 = __builtin_amdgcn_permlane16_swap(y32[0], y32[1], false, false);
  return make_uint4(x16[0], y16[0], x16[1], y16[1]);
}
// The same exchange through the LDS crossbar (ds_bpermute), for an epilogue whose
// register schedule measured faster with it (the rowwise fp8 dgu).
__device__ __forceinline__ uint4 span64_lds(uint2 lo, uint2 hi, int lane) {
  const int g = lane >> 4;
  const int s1 = (lane & 15) + 16 * ((2 * g) & 3), s2 = s1 + 16;
  const uint32_t l0 = __shfl(lo.x, s1), l1 = __shfl(lo.y, s1), l2 = __shfl(lo.x, s2), l3 = __shfl(lo.y, s2);
  const uint32_t h0 = __shfl(hi.x, s1), h1 = __shfl(hi.y, s1), h2 = __shfl(hi.x, s2), h3 = __shfl(hi.y, s2);
  return g < 2 ? make_uint4(l0, l1, l2, l3) : make_uint4(h0, h1, h2, h3);
}
__device__ __forceinline__ uint2 pack4(const float (&v)[4]) {
  return make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
}


// 16-byte chunks of a bf16 (uint16_t) or fp32 row: 8 or 4 elements widened to
// fp32, and packed back with the row type's rounding.
template <typename T> struct Chunk;
template <> struct Chunk<uint16_t> {
  static constexpr int kN = 8;
  static __device__ __forceinline__ void unpack(uint4 v, float (&f)[8]) {
    f[0] = bf_lo(v.x); f[1] = bf_hi(v.x); f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
    f[4] = bf_lo(v.z); f[5] = bf_hi(v.z); f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
  }
  static __device__ __forceinline__ uint4 pack(const float (&f)[8]) {
    return make_uint4(pack_bf2(f[0], f[1]), pack_bf2(f[2], f[3]), pack_bf2(f[4], f[5]), pack_bf2(f[6], f[7]));
  }
  static __device__ __forceinline__ float round(float f) { return round_bf(f); }
};
template <> struct Chunk<float> {
  static constexpr int kN = 4;
  static __device__ __forceinline__ void unpack(uint4 v, float (&f)[4]) {
    f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
  }
  static __device__ __forceinline__ uint4 pack(const float (&f)[4]) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
  }
  static __device__ __forceinline__ float round(float f) { return f; }
};

// ---------------------------------------------------------------------------
// Order-preserving map of fp32 onto uint32 used for top-k selection: larger
// key == larger value, -0.0 sorts below +0.0 and every NaN is the largest key.
// This is the radix order torch's GPU top-k selects in.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t radix_key(float v) {
  uint32_t x = __float_as_uint(v);
  uint32_t mask = (x & 0x80000000u) ? 0xffffffffu : 0x80000000u;
  return (v == v) ? (x ^ mask) : 0xffffffffu;
}

// ---------------------------------------------------------------------------
// Wavefront helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint64_t o = __shfl_xor(v, off);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Block-wide exclusive prefix sum over up to 4*blockDim.x int32 values held
// 4 per thread (thread t owns elements 4t..4t+3). `tmp` is LDS scratch of at
// least blockDim.x/64 ints. Returns the block total; `out` receives the
// exclusive prefixes. Must be called by every thread of the block.
__device__ __forceinline__ int block_exclusive_scan4(const int (&v)[4], int (&out)[4], int* tmp) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int local = v[0] + v[1] + v[2] + v[3];
  int incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  if (lane == 63) tmp[wv] = incl;
  __syncthreads();
  int wave_base = 0, total = 0;
  for (int w = 0; w < nw; ++w) {
    int s = tmp[w];
    if (w < wv) wave_base += s;
    total += s;
  }
  __syncthreads();
  int run = wave_base + incl - local;
  out[0] = run; run += v[0];
  out[1] = run; run += v[1];
  out[2] = run; run += v[2];
  out[3] = run;
  return total;
}

// Wave-cooperative sum of n <= 64 fp32 values (lane x holds value x, lanes
// >= n hold anything) in the association order of torch's GPU reduction of a
// short contiguous row (ATen Reduce.cuh): with bw = largest power of two <= n,
// thread x first forms v[x] + v[x+bw], then partials are combined by
// shfl_down with offsets 1, 2, 4, ... (a pairwise tree over adjacent
// threads). Returns the total on every lane.
__device__ __forceinline__ float wave_torch_row_sum(float v, int n) {
  const int lane = threadIdx.x & 63;
  int bw = 1;
  while (bw * 2 <= n) bw *= 2;
  float hi = __shfl_down(v, bw);
  float p = (lane + bw < n) ? (v + hi) : v;
  for (int off = 1; off < bw; off <<= 1) p = p + __shfl_down(p, off);
  return __shfl(p, 0);
}

}  // namespace moe
