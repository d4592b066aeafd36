// fp8 e4m3 grouped GEMMs for the SwiGLU experts on MI355X (CDNA4 fp8 MFMA).
//
// The reference's fp8 MoE path is torchao's Float8TrainingOpConfig applied to
// the experts (torchtitan/components/quantization/float8.py:260-288): dynamic
// rowwise scaling, fp8 grouped GEMMs with fp32 accumulation, bf16 outputs,
// token groups padded to 16 (quantization/__init__.py:37-40). This file
// restates that recipe for gfx950:
//
//  * quantizers (HBM-bound): x -> (q = e4m3fn(x / s), s = 2^-floor(log2(448 / max(amax, 1e-12))))
//      - moe_fp8_quant_rows: one scale per row of a [rows, K] tensor;
//      - moe_fp8_quant_cols_t: per expert, one scale per column b of an
//        [E, A, B] tensor, written transposed as [E, B, A];
//      - moe_fp8_quant_tokens_t: per expert token group, one scale per column c
//        of a [R, C] tensor, written transposed as [C, Rpad] with every group
//        starting at a multiple of 128 tokens (zero padded).
//    so that every GEMM below reads both operands contiguous along k.
//  * fp8 grouped GEMMs, C[m][n] = (sum_k qP[m][k] qQ[n][k]) * sP[m] * sQ[n],
//    on v_mfma_scale_f32_16x16x128_f8f6f4 (unit MX scales): forward gate_up
//    (with the SwiGLU epilogue) and down; backward dgu (dy . w2 with the
//    SwiGLU backward), dx (dg . w1 + du . w3, two scaled products added in
//    bf16), dw13 and dw2 (k = the expert's token group).
//
// Tiles: 256 x 256 outputs of eight 64 x 128 wave tiles, 128 k per stage,
// persistent workgroups.
// Operands reach LDS by direct-to-LDS copies (global_load_lds_dwordx4, one
// wave instruction = 8 rows x 128 bytes, coalesced) into row-major 128-byte
// rows with 16-byte chunk c of row r at c ^ ((r >> 1) & 7), which is
// conflict-free for the fragment reads; two stages, one barrier per k-step,
// copies waited for with explicit vmcnt. The copy stream runs through a
// workgroup's tiles one stage ahead of the MFMAs, across tile boundaries. Each lane's 32-byte MFMA fragment is
// chunks (lane >> 4) and 4 + (lane >> 4) of its row (any k order is valid as
// long as both operands share it). Rows past a segment and k past a padded
// token group are copied from a zero row.
//
// MXFP8 (torchao's MXFP8TrainingOpConfig, recipe "mxfp8_rceil", converted by
// torchtitan/components/quantization/mx.py:25-128; token groups padded to 32,
// quantization/__init__.py:36-40) uses the same kernels with one e8m0 scale
// per 32 consecutive k of every row:
//  * scale exponent e = clamp(ceil(log2(amax / 448)), -127, 127) + 127 (NaN
//    -> 255), elements q = e4m3fn(clamp(x * 2^(127 - e), +-448)), with x * 1
//    when e == 0 (torchao's RCEIL derivation);
//  * the MFMA applies the two scales itself: in the fragment layout above lane
//    group g holds k [16 g, +16) and [64 + 16 g, +16) of its row, and the
//    instruction's 32-k scale block b is k [32 b, 32 b + 32) with its scale
//    taken from lane group b of that row, so lane (row, g) passes the scale
//    of k-block 4 kt + g;
//  * scales reach LDS by direct-to-LDS copies next to the data: rows x 4
//    bytes (one dword = the 4 k-blocks of a 128-k stage) for row-grouped
//    operands, k-block x 16 rows for token-transposed ones.
#include "common.h"

namespace moe {
namespace fp8 {

typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kFp8Max = 448.0f;
constexpr int kPad = 128;  // token-group alignment of the token-transposed layouts (whole 128-byte lines)
constexpr int kMaxE = 1024;

// float -> float8_e4m3fn, round to nearest even, saturating at +-448.
__device__ __forceinline__ uint32_t e4m3(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t q;
  if (!(a < 448.0f)) {
    q = (a == a) ? 0x7eu : 0x7fu;  // saturate; NaN stays NaN
  } else if (a < 0.015625f) {        // below 2^-6: subnormal steps of 2^-9
    q = (uint32_t)rintf(a * 512.0f);
  } else {
    uint32_t u = __float_as_uint(a);
    u += 0x7ffffu + ((u >> 20) & 1u);  // round the mantissa to 3 bits, ties to even
    q = (u >> 20) - ((127u - 7u) << 3);
    q = q > 0x7eu ? 0x7eu : q;
  }
  return sign | q;
}

// The same conversion for four floats on the hardware (gfx950 v_cvt_pk_fp8_f32:
// OCP e4m3fn, round to nearest even) after fmed3 saturates them at +-448,
// packed little-endian. Checked against e4m3() on the GPU for every fp32 bit
// pattern: identical except NaN (which fmed3 turns into 448), so callers use it
// only for NaN-free data and keep e4m3() for the rest.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, -kFp8Max, kFp8Max),
                                                 __builtin_amdgcn_fmed3f(b, -kFp8Max, kFp8Max), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(c, -kFp8Max, kFp8Max),
                                                   __builtin_amdgcn_fmed3f(d, -kFp8Max, kFp8Max), lo, true);
}

// Nonzero when one of the eight bf16 values of v is a NaN: per 16-bit half,
// |h| + 0x7f carries into bit 15 exactly when |h| > 0x7f80.
__device__ __forceinline__ uint32_t has_nan8(uint4 v) {
  auto w = [](uint32_t x) { return (x & 0x7fff7fffu) + 0x007f007fu; };
  return (w(v.x) | w(v.y) | w(v.z) | w(v.w)) & 0x80008000u;
}

// true in every lane when no lane of the wave has a NaN (wave-uniform branch)
__device__ __forceinline__ bool wave_nan_free(uint32_t nan_flag) { return __ballot(nan_flag != 0u) == 0ull; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Rowwise scale of torchao's float8 MoE training (scales rounded down to powers of
// two): m = fp32(448 / max(amax, 1e-12)) formed in fp64, j = floor(log2 m) from m's
// exponent; returns the dequantization multiplier s = 2^-j, so x / s is exact and
// |x / s| <= 448 before the e4m3 rounding.
__device__ __forceinline__ float scale_of(float amax) {
  const float m = (float)(448.0 / fmax((double)amax, 1e-12));
  int e;
  (void)frexpf(m, &e);  // m = f 2^e with f in [0.5, 1)
  return ldexpf(1.0f, 1 - e);
}

constexpr int kMxBlock = 32;  // MXFP8 scaling block (k elements per e8m0 scale)
constexpr int kMxPad = 128;   // MXFP8 token-group alignment

// e8m0 exponent of an MX block from its amax (RCEIL):
// clamp(ceil(log2(amax / 448)), -127, 127) + 127, 255 for NaN.
__device__ __forceinline__ uint32_t mx_exponent(float amax) {
  const float d = amax / kFp8Max;
  if (d != d) return 255u;
  const uint32_t b = __float_as_uint(d);
  if (b >= 0x7f800000u) return 254u;
  const uint32_t ex = b >> 23, man = b & 0x7fffffu;
  if (ex == 0) return man > 0x400000u ? 1u : 0u;  // subnormal: above 2^-127 rounds up to 2^-126
  const uint32_t e = ex + (man != 0u);
  return e > 254u ? 254u : e;
}

// the element multiplier 2^(127 - e) (1 when e == 0)
__device__ __forceinline__ float mx_multiplier(uint32_t e) {
  if (e == 0) return 1.0f;
  if (e <= 253u) return __uint_as_float((254u - e) << 23);
  return __uint_as_float(0x400000u >> (e - 254u));  // 2^-127, 2^-128 (subnormal)
}

// ---------------------------------------------------------------------------
// quantizers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float amax8(uint4 v) {
  return fmaxf(fmaxf(fmaxf(fabsf(bf_lo(v.x)), fabsf(bf_hi(v.x))), fmaxf(fabsf(bf_lo(v.y)), fabsf(bf_hi(v.y)))),
               fmaxf(fmaxf(fabsf(bf_lo(v.z)), fabsf(bf_hi(v.z))), fmaxf(fabsf(bf_lo(v.w)), fabsf(bf_hi(v.w)))));
}

// fast: the wave's data holds no NaN (hardware conversion)
__device__ __forceinline__ uint2 mx_quant8(uint4 v, float f, bool fast) {
  if (fast)
    return make_uint2(e4m3x4(bf_lo(v.x) * f, bf_hi(v.x) * f, bf_lo(v.y) * f, bf_hi(v.y) * f),
                      e4m3x4(bf_lo(v.z) * f, bf_hi(v.z) * f, bf_lo(v.w) * f, bf_hi(v.w) * f));
  const uint32_t lo = e4m3(bf_lo(v.x) * f) | (e4m3(bf_hi(v.x) * f) << 8) | (e4m3(bf_lo(v.y) * f) << 16) |
                      (e4m3(bf_hi(v.y) * f) << 24);
  const uint32_t hi = e4m3(bf_lo(v.z) * f) | (e4m3(bf_hi(v.z) * f) << 8) | (e4m3(bf_lo(v.w) * f) << 16) |
                      (e4m3(bf_hi(v.w) * f) << 24);
  return make_uint2(lo, hi);
}

// q = e4m3fn(x / s): s is a power of two, so x * (1 / s) is the same exact scaling
__device__ __forceinline__ uint2 quant8(uint4 v, float s, bool fast) { return mx_quant8(v, 1.0f / s, fast); }


// One wave per row of x [rows, K] (K % 8 == 0). With CPL > 0 the row (up to
// 64 * CPL 16-byte chunks) stays in registers between the amax and the
// quantize step, so it is read once; CPL == 0 reads it twice.
template <int CPL>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x, int64_t rows, int K,
                                                         uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int cpr = K / 8;
  for (int64_t r = (int64_t)blockIdx.x * 4 + wv; r < rows; r += (int64_t)gridDim.x * 4) {
    const uint16_t* xr = x + r * K;
    uint8_t* qr = q + r * K;
    float amax = 0.f;
    uint32_t nan = 0;
    if constexpr (CPL > 0) {
      uint4 v[CPL];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < cpr ? *(const uint4*)(xr + c * 8) : make_uint4(0, 0, 0, 0);
        amax = fmaxf(amax, amax8(v[i]));
        nan |= has_nan8(v[i]);
      }
      const float s = scale_of(wave_max(amax));
      const bool fast = wave_nan_free(nan);
      if (lane == 0) scale[r] = s;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        if (c < cpr) *(uint2*)(qr + c * 8) = quant8(v[i], s, fast);
      }
    } else {
      for (int c = lane; c < cpr; c += 64) {
        const uint4 v = *(const uint4*)(xr + c * 8);
        amax = fmaxf(amax, amax8(v));
        nan |= has_nan8(v);
      }
      const float s = scale_of(wave_max(amax));
      const bool fast = wave_nan_free(nan);
      if (lane == 0) scale[r] = s;
      for (int c = lane; c < cpr; c += 64) *(uint2*)(qr + c * 8) = quant8(*(const uint4*)(xr + c * 8), s, fast);
    }
  }
}

// x [E][A][B] quantized along B, one scale per row (as quant_rows_kernel), with
// the column amax over A of every (e, b) on the side, for the transposed
// quantization of the same tensor (quant_cols_t_kernel with amax_in): the weights
// are then read twice per step instead of three times. Block (e, s) takes rows
// [s RB, s RB + RB) of expert e, one wave per row; each lane keeps the running
// maximum of its columns (|x|, NaN ignored as fmaxf does), the block's waves merge
// theirs in LDS, and one atomic max per column and block goes to col_amax (fp32
// bits of non-negative values order as unsigned integers; the caller zeroes it).
template <int CPL>
__global__ __launch_bounds__(256) void quant_rows_colamax_kernel(const uint16_t* __restrict__ x, int A, int B, int RB,
                                                                 uint8_t* __restrict__ q, float* __restrict__ scale,
                                                                 uint32_t* __restrict__ col_amax) {
  __shared__ uint32_t s_cm[64 * CPL * 8];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int cpr = B / 8;
  const int64_t e = blockIdx.y;
  const int a0 = blockIdx.x * RB, a1 = min(A, a0 + RB);
  for (int i = threadIdx.x; i < cpr * 8; i += blockDim.x) s_cm[i] = 0u;
  float cm[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k) cm[i][k] = 0.f;
  for (int a = a0 + wv; a < a1; a += 4) {
    const int64_t r = e * A + a;
    const uint16_t* xr = x + r * B;
    uint4 v[CPL];
    float amax = 0.f;
    uint32_t nan = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      v[i] = c < cpr ? *(const uint4*)(xr + c * 8) : make_uint4(0, 0, 0, 0);
      amax = fmaxf(amax, amax8(v[i]));
      nan |= has_nan8(v[i]);
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        cm[i][2 * k] = fmaxf(cm[i][2 * k], fabsf(bf_lo(w[k])));
        cm[i][2 * k + 1] = fmaxf(cm[i][2 * k + 1], fabsf(bf_hi(w[k])));
      }
    }
    const float s = scale_of(wave_max(amax));
    const bool fast = wave_nan_free(nan);
    if (lane == 0) scale[r] = s;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      if (c < cpr) *(uint2*)(q + r * B + c * 8) = quant8(v[i], s, fast);
    }
  }
  __syncthreads();  // s_cm cleared
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < cpr) {
#pragma unroll
      for (int k = 0; k < 8; ++k) atomicMax(&s_cm[c * 8 + k], __float_as_uint(cm[i][k]));
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < cpr * 8; i += blockDim.x) atomicMax(&col_amax[e * B + i], s_cm[i]);
}

// Rows gathered from another tensor (GATHER): row r of the operand is source row
// idx[r] of src (row stride ld), times scale[r] rounded to bf16 when scale is
// given (the expert permute x[token_idx] * score, read in place of its output).
// Source rows outside [0, n_src) read as zeros.
struct RowGather {
  const uint16_t* src = nullptr;
  const int64_t* idx = nullptr;
  const float* scale = nullptr;
  int64_t ld = 0, n_src = 0;
};

// v times s, rounded to bf16 (the permute's (x.float() * s).to(bf16))
__device__ __forceinline__ uint4 scale_chunk(uint4 v, float s) {
  float f[8];
  Chunk<uint16_t>::unpack(v, f);
#pragma unroll
  for (int k = 0; k < 8; ++k) f[k] = f[k] * s;
  return Chunk<uint16_t>::pack(f);
}

// x [R][C] with expert token groups (counts, consecutive in row order) quantized
// as quant_rows_kernel does with rows of K = C / P columns (piece p of row r
// scaled by scale[r P + p]), with the column amax of every (group, column) on the
// side, group_amax [E][C] (fp32 bits, atomic max; the caller zeroes it), for the
// token-transposed quantization of the same tensor (quant_tokens_t_kernel with
// amax_in), which then reads it once instead of twice. Block b takes rows
// [b RB, b RB + RB); for each group overlapping them, one wave per row keeps
// per-lane running column maxima (|x|, NaN ignored as fmaxf does), merged in LDS
// and sent with one atomic max per column when the block leaves the group. Rows
// past the last group are quantized row-wise only.
template <int CPL, int P, bool GATHER = false>
__global__ __launch_bounds__(256) void quant_rows_groupamax_kernel(const uint16_t* __restrict__ x,
                                                                   const int64_t* __restrict__ counts, int64_t R,
                                                                   int E, int C, int RB, uint8_t* __restrict__ q,
                                                                   float* __restrict__ scale,
                                                                   uint32_t* __restrict__ group_amax,
                                                                   RowGather gather) {
  __shared__ uint32_t s_cm[64 * CPL * 8];
  __shared__ int64_t s_end[kMaxE + 1];  // s_end[e]: end row of group e; s_end[E] = R
  __shared__ int s_tmp[8];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int cpr = C / 8, kc = cpr / P;  // 16-byte chunks per row and per piece
  {
    int cnt[4], st[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ee = threadIdx.x * 4 + i;
      const int64_t c = ee < E ? counts[ee] : 0;
      cnt[i] = c < 0 ? 0 : (int)(c > R ? R : c);
    }
    block_exclusive_scan4(cnt, st, s_tmp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ee = threadIdx.x * 4 + i;
      if (ee < E) s_end[ee] = min((int64_t)st[i] + cnt[i], R);
    }
    if (threadIdx.x == 0) s_end[E] = R;
  }
  for (int i = threadIdx.x; i < cpr * 8; i += blockDim.x) s_cm[i] = 0u;
  __syncthreads();
  const int64_t lo = (int64_t)blockIdx.x * RB, hi = min(R, lo + RB);
  if (lo >= hi) return;
  int e = 0, top = E;  // first group whose end is past lo (s_end is non-decreasing)
  while (e < top) {
    const int mid = (e + top) / 2;
    if (s_end[mid] > lo) top = mid; else e = mid + 1;
  }
  for (int64_t a = lo; a < hi && e <= E; ++e) {
    const int64_t b = min(hi, s_end[e]);  // rows [a, b) of group e (e == E: past the groups)
    if (b <= a) continue;
    float cm[CPL][8];
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
      for (int k = 0; k < 8; ++k) cm[i][k] = 0.f;
    for (int64_t r = a + wv; r < b; r += 4) {
      const uint16_t* xr = x + r * C;
      bool valid = true;
      float rs = 1.f;
      if constexpr (GATHER) {
        const int64_t j = gather.idx[r];
        valid = j >= 0 && j < gather.n_src;
        xr = gather.src + (valid ? j : 0) * gather.ld;
        if (gather.scale) rs = gather.scale[r];
      }
      uint4 v[CPL];
      float am[P];
#pragma unroll
      for (int p = 0; p < P; ++p) am[p] = 0.f;
      uint32_t nan = 0;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < cpr ? *(const uint4*)(xr + c * 8) : make_uint4(0, 0, 0, 0);
        if constexpr (GATHER) {
          if (!valid) v[i] = make_uint4(0, 0, 0, 0);
          else if (gather.scale) v[i] = scale_chunk(v[i], rs);
        }
        const float a8 = amax8(v[i]);
        if (P == 1 || c < kc) am[0] = fmaxf(am[0], a8);
        else am[P - 1] = fmaxf(am[P - 1], a8);
        nan |= has_nan8(v[i]);
        const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          cm[i][2 * k] = fmaxf(cm[i][2 * k], fabsf(bf_lo(w[k])));
          cm[i][2 * k + 1] = fmaxf(cm[i][2 * k + 1], fabsf(bf_hi(w[k])));
        }
      }
      float sp[P];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        sp[p] = scale_of(wave_max(am[p]));
        if (lane == 0) scale[r * P + p] = sp[p];
      }
      const bool fast = wave_nan_free(nan);
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        if (c < cpr) *(uint2*)(q + r * C + c * 8) = quant8(v[i], (P == 1 || c < kc) ? sp[0] : sp[P - 1], fast);
      }
    }
    if (e == E) break;
    // the block leaves group e: merge the waves' maxima, one atomic per column
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      if (c < cpr) {
#pragma unroll
        for (int k = 0; k < 8; ++k) atomicMax(&s_cm[c * 8 + k], __float_as_uint(cm[i][k]));
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < C; i += blockDim.x) {
      atomicMax(&group_amax[(int64_t)e * C + i], s_cm[i]);
      s_cm[i] = 0u;
    }
    __syncthreads();
    a = b;
  }
}

// Column amax over `n_rows` rows of a COLS-column slab (row stride ld elements)
// -> s_amax[COLS]; every thread of the 4 COLS-thread block calls it. Four independent 16-byte
// loads per thread are in flight per iteration.
template <int COLS>
__device__ __forceinline__ void slab_amax(const uint16_t* __restrict__ base, int64_t ld, int n_rows, float* s_red,
                                          float* s_amax) {
  const int t = threadIdx.x;
  constexpr int CPR = COLS / 8;
  const int ch = t % CPR, r0 = t / CPR;  // CPR chunks of 8 columns, 32 rows per sweep
  float m[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) m[i] = 0.f;
  for (int r = r0; r < n_rows; r += 128) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      v[u] = (r + 32 * u < n_rows) ? *(const uint4*)(base + (int64_t)(r + 32 * u) * ld + ch * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      m[0] = fmaxf(m[0], fabsf(bf_lo(v[u].x))); m[1] = fmaxf(m[1], fabsf(bf_hi(v[u].x)));
      m[2] = fmaxf(m[2], fabsf(bf_lo(v[u].y))); m[3] = fmaxf(m[3], fabsf(bf_hi(v[u].y)));
      m[4] = fmaxf(m[4], fabsf(bf_lo(v[u].z))); m[5] = fmaxf(m[5], fabsf(bf_hi(v[u].z)));
      m[6] = fmaxf(m[6], fabsf(bf_lo(v[u].w))); m[7] = fmaxf(m[7], fabsf(bf_hi(v[u].w)));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) s_red[(ch * 8 + i) * 33 + r0] = m[i];
  __syncthreads();
  if (t < COLS) {
    float a = 0.f;
    for (int j = 0; j < 32; ++j) a = fmaxf(a, s_red[t * 33 + j]);
    s_amax[t] = a;
  }
  __syncthreads();
}

constexpr int kTRows = 128;  // slab rows transposed per pass

// Quantizes a [n_rows x COLS] bf16 slab (row stride ld; COLS 64 or 128, a block of
// 4 COLS threads) transposed: output row b
// (slab column b) holds n_out values at out + b * ldo, rows >= n_rows zero
// (n_out a multiple of 16, and of 32 for MX; the token groups use 128).
//  * fp8 (MX false): column b scaled by s_col[b];
//  * MX: one e8m0 scale per (column b, 32-row block k) at sc + b * sc_b + k * sc_k;
//  * ROWS (MX): the same read also quantizes the slab along its columns (the
//    row-wise MX layout, blocks of 32 columns): row r's COLS values go to
//    qr + r * ldr and its COLS / 32 block scales to sr + r * ldsr.
// A pass moves 128 rows (four 16-byte loads per thread, double-buffered in
// registers so that two passes' loads are in flight) through s_tile
// (128 row-major rows of 2 COLS bytes, written with 16-byte stores, the 16-byte
// chunk c of row r at c ^ ((r / 16) % 8)). Each thread then quantizes two units
// of 16 rows of one column (2-byte reads; the swizzle keeps the eight row
// groups a wave reads at once in distinct banks) and stores their 16 bytes, so
// that 8 consecutive lanes write 128 contiguous bytes of one output row. The
// loads two passes ahead are issued as soon as the tile is in LDS. 128-column
// slabs (launched whenever the width allows) write the row-wise layout in whole
// 128-byte lines: 2-12 % faster than 64-column ones at the Kimi shapes.
// GATHER: the slab's rows are gathered (RowGather); the indices are loaded two
// passes ahead of the rows they address and the scale is applied when a pass is
// consumed, so neither waits behind the row loads in flight.
template <bool MX, bool ROWS, int COLS, bool GATHER = false>
__device__ __forceinline__ void slab_t_quant(const uint16_t* __restrict__ base, int64_t ld, int n_rows, int n_out,
                                             uint8_t* __restrict__ out, int64_t ldo, uint8_t* __restrict__ sc,
                                             int64_t sc_b, int64_t sc_k, const float* s_col, uint32_t* s_tile,
                                             uint8_t* __restrict__ qr = nullptr, int64_t ldr = 0,
                                             uint8_t* __restrict__ sr = nullptr, int64_t ldsr = 0,
                                             RowGather gather = RowGather{}, int shift = 0) {
  constexpr int T = 4 * COLS, CPR = COLS / 8;
  const int t = threadIdx.x;
  auto in_rows = [&](int row) { return row >= 0 && row < n_rows; };
  // Barriers wait for LDS only: __syncthreads() would also drain the global loads
  // of the passes ahead and the stores behind (its workgroup-scope fence is a
  // vmcnt(0)), which left one pass in flight. The tile's NaN flag is one word
  // per wave, written before and read after the second barrier of a pass (the
  // next pass's writes come after its first barrier, so one set of words does).
  __shared__ uint32_t s_wnan[T / 64];
  auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  uint4 va[4], vb[4];
  int64_t ia[4], ib[4];  // GATHER: source rows of the pass two ahead of va / vb
  float sa[4], sb[4];    // GATHER with scale: the row scales of the pass in va / vb
  // Every load is issued, rows outside the slab (and passes past its end) reading
  // a clamped row whose value is then dropped: with no load skipped on any path,
  // the compiler counts the loads in flight and waits for one pass's rows with
  // vmcnt(N) rather than vmcnt(0), which drained the pass ahead as well.
  // The rows' values are zeroed where they are consumed (zero_rows), not where they
  // are loaded: a select right after a load makes the load's wait immediate.
  auto clamp_row = [&](int row) { return row < 0 ? 0 : (row >= n_rows ? n_rows - 1 : row); };
  auto load_idx = [&](int64_t (&ix)[4], int a0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ix[i] = gather.idx[clamp_row(a0 + (t + i * T) / CPR)];
  };
  // GATHER: ok gets bit i when load i reads a row of the slab with a source row in range
  auto load = [&](uint4 (&v)[4], const int64_t (&ix)[4], float (&sv)[4], uint32_t& ok, int a0) {
    ok = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + i * T;
      const int r = c / CPR, ch = c % CPR;
      if constexpr (GATHER) {
        const bool in = in_rows(a0 + r) && ix[i] >= 0 && ix[i] < gather.n_src;
        ok |= in ? 1u << i : 0u;
        v[i] = *(const uint4*)(gather.src + (in ? ix[i] : 0) * gather.ld + ch * 8);
        if (gather.scale) sv[i] = gather.scale[clamp_row(a0 + r)];
      } else {
        v[i] = *(const uint4*)(base + (int64_t)clamp_row(a0 + r) * ld + ch * 8);
      }
    }
  };
  auto zero_rows = [&](uint4 (&v)[4], uint32_t ok, int a0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool in = GATHER ? ((ok >> i) & 1u) != 0u : in_rows(a0 + (t + i * T) / CPR);
      if (!in) v[i] = make_uint4(0, 0, 0, 0);
    }
  };
  auto apply_scales = [&](uint4 (&v)[4], const float (&sv)[4], int a0) {
    if constexpr (GATHER) {
      if (!gather.scale) return;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!in_rows(a0 + (t + i * T) / CPR)) continue;
        v[i] = scale_chunk(v[i], sv[i]);
      }
    }
  };
  // one pass of 128 rows held in v; v is reloaded with the pass two ahead as soon
  // as it is in LDS, so two passes' loads are in flight while one is transposed
  auto pass = [&](uint4 (&v)[4], int64_t (&ix)[4], float (&sv)[4], uint32_t& ok, int a0) {
    zero_rows(v, ok, a0);
    apply_scales(v, sv, a0);
    const uint32_t nan = has_nan8(v[0]) | has_nan8(v[1]) | has_nan8(v[2]) | has_nan8(v[3]);
    if constexpr (ROWS) {
      const bool rows_fast = wave_nan_free(nan);
      // lanes t, t ^ 1, t ^ 2, t ^ 3 hold the four 8-column chunks of one 32-column block
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = t + i * T;
        const int r = c / CPR, ch = c % CPR;
        float a = amax8(v[i]);
        a = fmaxf(a, __shfl_xor(a, 1));
        a = fmaxf(a, __shfl_xor(a, 2));
        const uint32_t e = mx_exponent(a);
        if (in_rows(a0 + r)) {
          *(uint2*)(qr + (int64_t)(a0 + r) * ldr + ch * 8) = mx_quant8(v[i], mx_multiplier(e), rows_fast);
          if ((ch & 3) == 0) sr[(int64_t)(a0 + r) * ldsr + (ch >> 2)] = (uint8_t)e;
        }
      }
    }
    lds_barrier();  // every thread's LDS reads of the previous pass are done
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + i * T;
      const int r = c / CPR;
      *(uint4*)(s_tile + r * (COLS / 2) + (((c % CPR) ^ ((r >> 4) & 7)) * 4)) = v[i];
    }
    {
      const bool wave_nan = !wave_nan_free(nan);
      if ((t & 63) == 0) s_wnan[t >> 6] = wave_nan ? 1u : 0u;
    }
    lds_barrier();  // the tile and the flags are in LDS
    uint32_t any_nan = 0;
#pragma unroll
    for (int w = 0; w < T / 64; ++w) any_nan |= s_wnan[w];
    const bool fast = any_nan == 0u;  // block-uniform: the tile holds no NaN
    load(v, ix, sv, ok, a0 + 2 * kTRows);
    if constexpr (GATHER) load_idx(ix, a0 + 4 * kTRows);
    // unit (column cc, rows 16 kq .. 16 kq + 15 of the pass): 8 consecutive lanes cover one
    // output row's 128 bytes, so every store instruction writes 8 rows x 128 contiguous bytes
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int u = t + T * h;
      const int cc = u >> 3, kq = u & 7;
      const int rb = a0 + 16 * kq;
      // column cc of pass rows 16 kq + s sits in chunk (cc / 8) ^ kq of its row
      const uint16_t* xs = (const uint16_t*)s_tile + (16 * kq) * COLS + (((cc >> 3) ^ kq) * 8) + (cc & 7);
      float xv[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) xv[k] = bf2f(xs[COLS * k]);
      float f;
      uint32_t e = 0;
      if constexpr (MX) {
        float am = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) am = fmaxf(am, fabsf(xv[k]));
        am = fmaxf(am, __shfl_xor(am, 1));  // the 32-row block is lanes kq, kq ^ 1
        e = mx_exponent(am);
        f = mx_multiplier(e);
      } else {
        f = 1.0f / s_col[cc];  // s is a power of two: x * f is x / s exactly
      }
      uint32_t o[4];
      if (fast) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          o[q] = e4m3x4(xv[4 * q] * f, xv[4 * q + 1] * f, xv[4 * q + 2] * f, xv[4 * q + 3] * f);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          o[q] = 0;
#pragma unroll
          for (int bq = 0; bq < 4; ++bq) o[q] |= e4m3(xv[4 * q + bq] * f) << (8 * bq);
        }
      }
      if (rb >= 0 && rb < n_out) {
        *(uint4*)(out + (int64_t)cc * ldo + rb) = make_uint4(o[0], o[1], o[2], o[3]);
        if constexpr (MX)
          if ((kq & 1) == 0) sc[(int64_t)cc * sc_b + (int64_t)(rb / kMxBlock) * sc_k] = (uint8_t)e;
      }
    }
  };
  // passes start `shift` rows before the slab (rows < 0 are neither loaded nor
  // stored), so that with shift = the output offset mod 128 every pass writes
  // whole 128-byte lines of each output row
  const int b0 = -shift;
  if constexpr (GATHER) {
    load_idx(ia, b0);
    load_idx(ib, b0 + kTRows);
  }
  uint32_t oka, okb;
  load(va, ia, sa, oka, b0);
  if constexpr (GATHER) load_idx(ia, b0 + 2 * kTRows);
  load(vb, ib, sb, okb, b0 + kTRows);
  if constexpr (GATHER) load_idx(ib, b0 + 3 * kTRows);
  for (int a0 = b0; a0 < n_out; a0 += 2 * kTRows) {
    pass(va, ia, sa, oka, a0);
    if (a0 + kTRows < n_out) pass(vb, ib, sb, okb, a0 + kTRows);
  }
}

// x [E][A][B] -> q rows (e, b) of A values at q + e * q_estride + b * q_ld, and
// scale[e * s_estride + b] = amax over A. Block per (e, COLS columns). With
// amax_in (the column amax [E][B] already known, from quant_rows_colamax_kernel)
// the amax pass is skipped and x is read once.
template <int COLS>
__global__ __launch_bounds__(4 * COLS) void quant_cols_t_kernel(const uint16_t* __restrict__ x, int A, int B,
                                                           uint8_t* __restrict__ q, int64_t q_estride, int64_t q_ld,
                                                           float* __restrict__ scale, int64_t s_estride,
                                                           const float* __restrict__ amax_in) {
  __shared__ float s_red[COLS * 33];
  __shared__ float s_amax[COLS];
  __shared__ __attribute__((aligned(16))) uint32_t s_tile[kTRows * (COLS / 2)];
  const int nb = B / COLS;
  const int64_t e = blockIdx.x / nb;
  const int b0 = (blockIdx.x % nb) * COLS;
  const uint16_t* base = x + e * A * (int64_t)B + b0;
  if (amax_in) {
    if (threadIdx.x < COLS) s_amax[threadIdx.x] = amax_in[e * B + b0 + threadIdx.x];
    __syncthreads();
  } else {
    slab_amax<COLS>(base, B, A, s_red, s_amax);
  }
  if (threadIdx.x < COLS) {
    const float s = scale_of(s_amax[threadIdx.x]);
    s_amax[threadIdx.x] = s;
    scale[e * s_estride + b0 + threadIdx.x] = s;
  }
  __syncthreads();
  slab_t_quant<false, false, COLS>(base, B, A, A, q + e * q_estride + b0 * q_ld, q_ld, nullptr, 0, 0, s_amax, s_tile);
}

// x [R][C] with expert token groups (counts) -> q [C][Rpad] (group e at the
// 128-aligned offset pstart_e, zero padded to ceil128(count_e)), scale [E][C].
// Block per (e, COLS columns); empty groups exit. With amax_in (the column amax
// [E][C] of every group already known, from quant_rows_groupamax_kernel) the
// amax pass is skipped and x is read once.
template <int COLS, bool GATHER = false>
__global__ __launch_bounds__(4 * COLS) void quant_tokens_t_kernel(const uint16_t* __restrict__ x, const int64_t* __restrict__ counts,
                                                             int64_t R, int E, int C, int64_t Rpad,
                                                             uint8_t* __restrict__ q, float* __restrict__ scale,
                                                             const float* __restrict__ amax_in, RowGather gather) {
  __shared__ float s_red[COLS * 33];
  __shared__ float s_amax[COLS];
  __shared__ __attribute__((aligned(16))) uint32_t s_tile[kTRows * (COLS / 2)];
  __shared__ int s_tmp[8];
  __shared__ int s_seg[2];
  // slab-major: the blocks running together share column slabs (1-4 % faster
  // than expert-major at the Kimi shapes)
  const int e = blockIdx.x % E;
  const int c0 = (blockIdx.x / E) * COLS;
  {
    int cnt[4], pc[4], st[4], pst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ee = threadIdx.x * 4 + i;
      const int64_t c = ee < E ? counts[ee] : 0;
      cnt[i] = c < 0 ? 0 : (int)(c > R ? R : c);
      pc[i] = (cnt[i] + kPad - 1) / kPad * kPad;
    }
    block_exclusive_scan4(cnt, st, s_tmp);
    block_exclusive_scan4(pc, pst, s_tmp);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (threadIdx.x * 4 + i == e) { s_seg[0] = st[i]; s_seg[1] = pst[i]; s_red[0] = __int_as_float(cnt[i]); }
    __syncthreads();
  }
  const int seg0 = s_seg[0], pstart = s_seg[1];
  int n = __float_as_int(s_red[0]);
  __syncthreads();
  if ((int64_t)seg0 + n > R) n = (int)(R - seg0 > 0 ? R - seg0 : 0);
  const int n_out = (n + kPad - 1) / kPad * kPad;
  if (n == 0 || (int64_t)pstart + n_out > Rpad) return;
  const uint16_t* base = GATHER ? nullptr : x + (int64_t)seg0 * C + c0;
  if constexpr (GATHER) {  // this slab's rows and columns of the gathered source
    gather.src += c0;
    gather.idx += seg0;
    if (gather.scale) gather.scale += seg0;
  }
  if (GATHER || amax_in) {  // a gathered operand comes with its amax
    if (threadIdx.x < COLS) s_amax[threadIdx.x] = amax_in[(int64_t)e * C + c0 + threadIdx.x];
    __syncthreads();
  } else {
    slab_amax<COLS>(base, C, n, s_red, s_amax);
  }
  if (threadIdx.x < COLS) {
    const float s = scale_of(s_amax[threadIdx.x]);
    s_amax[threadIdx.x] = s;
    scale[(int64_t)e * C + c0 + threadIdx.x] = s;
  }
  __syncthreads();
  slab_t_quant<false, false, COLS, GATHER>(base, C, n, n_out, q + (int64_t)c0 * Rpad + pstart, Rpad, nullptr, 0, 0,
                                           s_amax, s_tile, nullptr, 0, nullptr, 0, gather, pstart % 128);
}

// ---------------------------------------------------------------------------
// MXFP8 quantizers
// ---------------------------------------------------------------------------


// x viewed as n_chunks 16-byte chunks of 8 bf16 (rows of K, K % 32 == 0): four
// consecutive lanes hold one 32-element block, reduce its amax by shuffles
// and write one e8m0 byte (block index = chunk / 4, i.e. scale [rows][K/32]).
// Four chunks per thread are loaded before any is processed.
__global__ __launch_bounds__(256) void mx_quant_rows_kernel(const uint4* __restrict__ x, int64_t n_chunks,
                                                            uint2* __restrict__ q, uint8_t* __restrict__ scale) {
  const int64_t S = (int64_t)gridDim.x * 256;
  for (int64_t c0 = (int64_t)blockIdx.x * 256 + threadIdx.x; c0 - threadIdx.x < n_chunks; c0 += 4 * S) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = c0 + u * S;
      v[u] = c < n_chunks ? x[c] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = c0 + u * S;
      float a = amax8(v[u]);
      a = fmaxf(a, __shfl_xor(a, 1));
      a = fmaxf(a, __shfl_xor(a, 2));
      const uint32_t e = mx_exponent(a);
      const bool fast = wave_nan_free(has_nan8(v[u]));
      if (c < n_chunks) {
        q[c] = mx_quant8(v[u], mx_multiplier(e), fast);
        if ((c & 3) == 0) scale[c >> 2] = (uint8_t)e;
      }
    }
  }
}

// x [E][A][B] -> q rows (e, b) of A values at q + e * q_estride + b * q_ld, and
// their A/32 scales at s + e * s_estride + b * s_ld. Block per (e, COLS columns).
template <int COLS>
__global__ __launch_bounds__(4 * COLS) void mx_quant_cols_t_kernel(const uint16_t* __restrict__ x, int A, int B,
                                                              uint8_t* __restrict__ q, int64_t q_estride,
                                                              int64_t q_ld, uint8_t* __restrict__ s,
                                                              int64_t s_estride, int64_t s_ld) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tile[kTRows * (COLS / 2)];
  const int nb = B / COLS;
  const int64_t e = blockIdx.x / nb;
  const int b0 = (blockIdx.x % nb) * COLS;
  slab_t_quant<true, false, COLS>(x + e * A * (int64_t)B + b0, B, A, A, q + e * q_estride + b0 * q_ld, q_ld,
                            s + e * s_estride + b0 * s_ld, s_ld, 1, nullptr, s_tile);
}

// Both MX layouts of x [E][A][B] from one read: the row-wise one (q_r [E][A][B],
// s_r [E][A][B / 32], as mx_quant_rows on [E A, B]) and the transposed one of
// mx_quant_cols_t. Block per (e, COLS columns).
template <int COLS>
__global__ __launch_bounds__(4 * COLS) void mx_dual_cols_kernel(const uint16_t* __restrict__ x, int A, int B,
                                                           uint8_t* __restrict__ q, int64_t q_estride, int64_t q_ld,
                                                           uint8_t* __restrict__ s, int64_t s_estride, int64_t s_ld,
                                                           uint8_t* __restrict__ qr, uint8_t* __restrict__ sr) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tile[kTRows * (COLS / 2)];
  const int nb = B / COLS;
  const int64_t e = blockIdx.x / nb;
  const int b0 = (blockIdx.x % nb) * COLS;
  const int64_t row0 = e * A;  // first row of expert e in the [E A, B] view
  slab_t_quant<true, true, COLS>(x + row0 * B + b0, B, A, A, q + e * q_estride + b0 * q_ld, q_ld,
                           s + e * s_estride + b0 * s_ld, s_ld, 1, nullptr, s_tile, qr + row0 * B + b0, B,
                           sr + row0 * (B / kMxBlock) + b0 / kMxBlock, B / kMxBlock);
}

// x [R][C] with expert token groups (counts) -> q [C][Rpad] (group e at the
// 128-aligned offset pstart_e, zero padded to ceil128(count_e)) and the scales
// k-block major, s [Rpad / 32][C]. Block per (e, COLS columns); empty groups exit.
// With ROWS, the same read also writes the row-wise layout of the group's rows
// (qr [R][C], sr [R][C / 32]).
template <bool ROWS, int COLS, bool GATHER = false>
__global__ __launch_bounds__(4 * COLS) void mx_quant_tokens_t_kernel(const uint16_t* __restrict__ x,
                                                                const int64_t* __restrict__ counts, int64_t R, int E,
                                                                int C, int64_t Rpad, uint8_t* __restrict__ q,
                                                                uint8_t* __restrict__ s, uint8_t* __restrict__ qr,
                                                                uint8_t* __restrict__ sr, RowGather gather) {
  __shared__ __attribute__((aligned(16))) uint32_t s_tile[kTRows * (COLS / 2)];
  __shared__ int s_tmp[8];
  __shared__ int s_seg[3];
  // slab-major: the blocks running together share column slabs (1-4 % faster
  // than expert-major at the Kimi shapes)
  const int e = blockIdx.x % E;
  const int c0 = (blockIdx.x / E) * COLS;
  {
    int cnt[4], pc[4], st[4], pst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ee = threadIdx.x * 4 + i;
      const int64_t c = ee < E ? counts[ee] : 0;
      cnt[i] = c < 0 ? 0 : (int)(c > R ? R : c);
      pc[i] = (cnt[i] + kMxPad - 1) / kMxPad * kMxPad;
    }
    block_exclusive_scan4(cnt, st, s_tmp);
    block_exclusive_scan4(pc, pst, s_tmp);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (threadIdx.x * 4 + i == e) { s_seg[0] = st[i]; s_seg[1] = pst[i]; s_seg[2] = cnt[i]; }
    __syncthreads();
  }
  const int seg0 = s_seg[0], pstart = s_seg[1];
  int n = s_seg[2];
  if ((int64_t)seg0 + n > R) n = (int)(R - seg0 > 0 ? R - seg0 : 0);
  const int n_out = (n + kMxPad - 1) / kMxPad * kMxPad;
  if (e == E - 1 && (int64_t)pstart + n_out <= Rpad) {
    // The columns past the last group, up to Rpad, belong to no group: zero them
    // (and their scale rows) so that every byte of q and s is defined. Both ends
    // are multiples of 32, so the rows' tails take 16-byte stores.
    const int64_t end = (int64_t)pstart + n_out;
    const int64_t tail16 = (Rpad - end) / 16;
    for (int64_t i = threadIdx.x; i < COLS * tail16; i += 4 * COLS) {
      const int64_t c = i / tail16, j = i - c * tail16;
      *(uint4*)(q + (c0 + c) * Rpad + end + 16 * j) = make_uint4(0u, 0u, 0u, 0u);
    }
    if (threadIdx.x < COLS)
      for (int64_t br = end / kMxBlock; br < Rpad / kMxBlock; ++br) s[br * C + c0 + threadIdx.x] = 0;
  }
  if (n == 0 || (int64_t)pstart + n_out > Rpad) return;
  if constexpr (GATHER) {  // this slab's rows and columns of the gathered source
    gather.src += c0;
    gather.idx += seg0;
    if (gather.scale) gather.scale += seg0;
  }
  slab_t_quant<true, ROWS, COLS, GATHER>(GATHER ? nullptr : x + (int64_t)seg0 * C + c0, C, n, n_out,
                                 q + (int64_t)c0 * Rpad + pstart, Rpad, s + (int64_t)(pstart / kMxBlock) * C + c0, 1, C,
                                 nullptr, s_tile, ROWS ? qr + (int64_t)seg0 * C + c0 : nullptr, C,
                                 ROWS ? sr + (int64_t)seg0 * (C / kMxBlock) + c0 / kMxBlock : nullptr, C / kMxBlock,
                                 gather, pstart % 128);
}

// ---------------------------------------------------------------------------
// fp8 grouped GEMM
// ---------------------------------------------------------------------------
enum Mode : int { kGateUp = 0, kDown = 1, kDgu = 2, kDx = 3, kDw13 = 4, kDw2 = 5 };

struct Params {
  const int64_t* counts;
  int64_t R, Rpad;
  int E, D, H;
  const uint8_t* qp;  // P operand (fp8, k-contiguous rows)
  const uint8_t* qq;  // Q operand
  const uint8_t* qq2; // second Q operand (w3 for gate_up)
  const float* sp;    // P scales
  const float* sq;    // Q scales
  const float* sq2;   // second Q scales
  const uint16_t* g;  // saved g, u for the SwiGLU backward
  const uint16_t* u;
  uint16_t* o0;  // outputs (mode dependent)
  uint16_t* o1;
  uint16_t* o2;
  const uint8_t* ep;   // MXFP8: e8m0 scales of P, Q and the second Q operand
  const uint8_t* eq;
  const uint8_t* eq2;
};

#define LDSP __attribute__((address_space(3)))
// One wave-wide direct-to-LDS copy: lane i's 16 bytes at g land at LDS byte
// address lds + 16 i; issued as inline asm and waited for with vmcnt.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" :: "v"(g), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* ptr) { return (uint32_t)(size_t)((LDSP const uint8_t*)ptr); }

// Row-major LDS tile with 128-byte rows (one 128-k stage of fp8): byte offset of
// 16-byte chunk c of row r; conflict-free for fragment reads of 16 rows.
__device__ __forceinline__ int rm_off(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// One wave-wide 4-byte direct-to-LDS copy: lane i's dword lands at lds + 4 i.
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dword %0, off" :: "v"(g), "{m0}"(lds) : "memory");
}

__device__ const uint4 kZeroRow[64] = {};  // source of zero rows and k past a segment
// e8m0 127 (= 1.0) scales for rows past a segment and k-blocks past a group
__device__ const uint4 kUnitScales[1] = {{0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu}};


// NW waves as WGM x (NW / WGM) wave tiles of (16 TM) x (16 TN), NS LDS stages of
// 128 k, OCC workgroups per CU. One stream of copy stages runs through this
// workgroup's tiles NS - 1 stages ahead of the MFMAs, across tile boundaries,
// so the next tile's first stages are in flight during this tile's epilogue.
// MX: e8m0 block scales (p.ep / p.eq / p.eq2) applied by the MFMA instead of
// the fp32 row scales of the epilogues; token groups aligned to 32; BM = BN =
// 32 NW and two stages (the scale copies assume them).
template <int MODE, int NW, int WGM, int TM, int TN, int NS, int OCC, bool MX>
__global__ __launch_bounds__(NW * 64, OCC) void fp8_gemm_kernel(Params p) {
  constexpr bool kRowGrouped = MODE <= kDx;
  constexpr int WGN = NW / WGM;
  constexpr int WM = TM * 16, WN = TN * 16, BM = WGM * WM, BN = WGN * WN;
  constexpr int CPW_P = BM / 8 / NW, CPW_Q = BN / 8 / NW;  // 1 KB copies (8 rows x 128 B) per wave and stage
  constexpr int CPW = CPW_P + CPW_Q;
  constexpr int PAD = MX ? kMxPad : kPad;
  static_assert(CPW_P * 8 * NW == BM && CPW_Q * 8 * NW == BN && CPW <= 30, "copies per wave");
  static_assert(NS == 2 || NS == 3, "stages");
  static_assert(!MX || (BM == 32 * NW && BN == 32 * NW && NS == 2),
                "the MX scale copies assume BM = BN = 32 NW (one dword per row and wave lane) and two stages");
  static_assert(TN % 2 == 0 && (MODE != kGateUp || TN % 4 == 0), "epilogue block pairs");
  // B fragments prefetched one 16-column block ahead where that measured faster in the
  // fp8 and MXFP8 layer steps at 32768 Kimi tokens (rowwise: gate_up -1.5 %, down -1 %,
  // dx -2.5 %, dgu +0.5 %; MX: gate_up -1.2 %, dgu -1.3 %, dx -1.5 %, dW +1.6-2 %)
  constexpr bool kPrefetchB = MX ? (MODE == kGateUp || MODE == kDgu || MODE == kDx)
                                 : (MODE == kGateUp || MODE == kDown || MODE == kDx);
  __shared__ __attribute__((aligned(1024))) uint8_t sP[NS][BM * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t sQ[NS][BN * 128];
  // MX scales of a stage: row-grouped, P row m's 4 k-blocks at 4 m and Q row n's
  // at 4 BM + 4 n; token-transposed, k-block j of P row m at BM j + m, of Q
  // row n at 4 BM + BN j + n
  __shared__ __attribute__((aligned(16))) uint8_t sS[NS][MX ? 4 * (BM + BN) : 16];
  __shared__ int s_seg[kMaxE + 1];
  __shared__ int s_pst[kMaxE + 1];
  __shared__ int s_tile[kMaxE + 1];
  __shared__ int s_tmp[8];

  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv / WGN, wn = wv % WGN;
  const int E = p.E, D = p.D, H = p.H;
  int Ntot = 0, Kfix = 0, Mfix = 0;
  if (MODE == kGateUp) { Ntot = 2 * H; Kfix = D; }
  if (MODE == kDown) { Ntot = D; Kfix = H; }
  if (MODE == kDgu) { Ntot = H; Kfix = D; }
  if (MODE == kDx) { Ntot = D; Kfix = 2 * H; }
  if (MODE == kDw13) { Ntot = D; Mfix = 2 * H; }
  if (MODE == kDw2) { Ntot = H; Mfix = D; }
  const int NT = Ntot / BN;
  const int MT = kRowGrouped ? 0 : Mfix / BM;
  {
    int cnt[4], tl[4], seg[4], pc[4], pst[4], tst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      const int64_t c = (e < E) ? p.counts[e] : 0;
      cnt[i] = c < 0 ? 0 : (c > p.R ? (int)p.R : (int)c);
    }
    {
      int pre[4];
      block_exclusive_scan4(cnt, pre, s_tmp);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t lo = pre[i] < p.R ? pre[i] : p.R;
        const int64_t hi = (int64_t)pre[i] + cnt[i] < p.R ? (int64_t)pre[i] + cnt[i] : p.R;
        cnt[i] = (int)(hi - lo);
        pc[i] = (cnt[i] + PAD - 1) / PAD * PAD;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      tl[i] = (e < E) ? (kRowGrouped ? ((cnt[i] + BM - 1) / BM) * NT : MT * NT) : 0;
    }
    const int rtot = block_exclusive_scan4(cnt, seg, s_tmp);
    const int ptot = block_exclusive_scan4(pc, pst, s_tmp);
    const int ttot = block_exclusive_scan4(tl, tst, s_tmp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      if (e < E) { s_seg[e] = seg[i]; s_pst[e] = pst[i]; s_tile[e] = tst[i]; }
    }
    if (tid == 0) { s_seg[E] = rtot; s_pst[E] = ptot; s_tile[E] = ttot; }
    __syncthreads();
  }
  if (!kRowGrouped && (int64_t)s_pst[E] > p.Rpad) return;  // inconsistent padding: nothing is read out of bounds
  const int total_tiles = s_tile[E];
  const int G = gridDim.x;
  const int lb = (G % 8 == 0) ? ((int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3)) : (int)blockIdx.x;

  // ks: bytes of k the token-transposed stages start before the group (pst0 mod 128,
  // masked), so that every stage reads whole 128-byte lines
  struct TileRef { int e, seg0, seg1, pst0, mt, nt, klen, nk, ks; };
  auto decode = [&](int t) {
    TileRef r;
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_tile[mid] <= t) lo = mid; else hi = mid - 1;
    }
    r.e = lo;
    const int local = t - s_tile[lo];
    r.seg0 = s_seg[lo];
    r.seg1 = s_seg[lo + 1];
    r.pst0 = s_pst[lo];
    if (kRowGrouped) {
      const int mtiles = (r.seg1 - r.seg0 + BM - 1) / BM;
      r.nt = local / mtiles;
      r.mt = local - r.nt * mtiles;
    } else {
      r.nt = local / MT;
      r.mt = local - r.nt * MT;
    }
    r.klen = kRowGrouped ? Kfix : (s_pst[lo + 1] - r.pst0);  // bytes of k
    r.ks = kRowGrouped ? 0 : r.pst0 % 128;
    r.nk = (r.klen + r.ks + 127) / 128;
    return r;
  };

  // ---- copy sources of the tile being copied: lane i of copy c fills row 8 c + i / 8,
  // 16-byte chunk (i % 8), loading global chunk (i % 8) ^ ((row >> 1) & 7) of that row ----
  const int crow = lane >> 3;
  const uint8_t* srcP[CPW_P];
  const uint8_t* srcQ[CPW_Q];
  bool okP[CPW_P];
  int chP[CPW_P], chQ[CPW_Q];
#pragma unroll
  for (int b = 0; b < CPW_P; ++b) chP[b] = ((lane & 7) ^ ((((wv * CPW_P + b) * 8 + crow) >> 1) & 7)) * 16;
#pragma unroll
  for (int b = 0; b < CPW_Q; ++b) chQ[b] = ((lane & 7) ^ ((((wv * CPW_Q + b) * 8 + crow) >> 1) & 7)) * 16;
  // MX scale copy source of this lane. Row-grouped: one dword copy per wave, the
  // first NW / 2 waves P rows 64 wv + lane, the others Q rows. Token-transposed:
  // one 16-byte copy by each lane gl = 64 wv + lane < (BM + BN) / 4 (the first NW / 4
  // waves), gl < BM / 4 P, the rest Q, each 16 rows of one k-block kbS of the stage.
  const uint8_t* srcS = nullptr;
  bool okS = false;
  int64_t kstrideS = 0;
  int kbS = 0;
  auto setup = [&](const TileRef& r) {
    const int64_t e64 = r.e;
    const int row0 = r.seg0 + r.mt * BM;
#pragma unroll
    for (int b = 0; b < CPW_P; ++b) {
      const int m = (wv * CPW_P + b) * 8 + crow;
      if (kRowGrouped) {
        const int rr = row0 + m;
        okP[b] = rr < r.seg1;
        srcP[b] = p.qp + (int64_t)rr * Kfix + chP[b];
      } else {
        okP[b] = true;
        srcP[b] = p.qp + (int64_t)(r.mt * BM + m) * p.Rpad + (r.pst0 - r.ks) + chP[b];
      }
    }
#pragma unroll
    for (int b = 0; b < CPW_Q; ++b) {
      const int n = (wv * CPW_Q + b) * 8 + crow;
      const uint8_t* rowp;
      if (MODE == kGateUp) {
        const int blk = n >> 4;
        const int hc = r.nt * (BN / 2) + (blk >> 1) * 16 + (n & 15);
        rowp = ((blk & 1) ? p.qq2 : p.qq) + (e64 * H + hc) * (int64_t)D;
      } else if (MODE == kDown) {
        rowp = p.qq + (e64 * D + r.nt * BN + n) * (int64_t)H;
      } else if (MODE == kDgu) {
        rowp = p.qq + (e64 * H + r.nt * BN + n) * (int64_t)D;
      } else if (MODE == kDx) {
        rowp = p.qq + (e64 * D + r.nt * BN + n) * (int64_t)(2 * H);
      } else {
        rowp = p.qq + (int64_t)(r.nt * BN + n) * p.Rpad + (r.pst0 - r.ks);
      }
      srcQ[b] = rowp + chQ[b];
    }
    if (MX) {
      if (kRowGrouped) {
        const int kb_row = Kfix / kMxBlock;  // scale bytes per row
        if (wv < NW / 2) {
          const int rr = row0 + wv * 64 + lane;
          okS = rr < r.seg1;
          srcS = p.ep + (int64_t)rr * kb_row;
        } else {
          const int n = (wv - NW / 2) * 64 + lane;
          okS = true;
          int64_t qrow;
          const uint8_t* base = p.eq;
          if (MODE == kGateUp) {
            const int blk = n >> 4;
            qrow = e64 * H + r.nt * (BN / 2) + (blk >> 1) * 16 + (n & 15);
            if (blk & 1) base = p.eq2;
          } else if (MODE == kDown) {
            qrow = e64 * D + r.nt * BN + n;
          } else if (MODE == kDgu) {
            qrow = e64 * H + r.nt * BN + n;
          } else {
            qrow = e64 * D + r.nt * BN + n;
          }
          srcS = base + qrow * kb_row;
        }
      } else {
        const int gl = wv * 64 + lane;
        const bool isP = gl < BM / 4;
        const int sub = isP ? gl : gl - BM / 4;
        const int cpk = isP ? BM / 16 : BN / 16;  // 16-byte chunks per k-block
        kbS = sub / cpk;
        const int64_t kb0 = (r.pst0 - r.ks) / kMxBlock + kbS;
        kstrideS = isP ? Mfix : Ntot;
        srcS = (isP ? p.ep + kb0 * Mfix + r.mt * BM : p.eq + kb0 * Ntot + r.nt * BN) + (sub % cpk) * 16;
      }
    }
  };
  // stage kt of tile r into LDS buffer s
  auto issue = [&](const TileRef& r, int kt, int s) {
    const int k0 = kt * 128;
#pragma unroll
    for (int b = 0; b < CPW_P; ++b) {
      const int kk = k0 + chP[b] - r.ks;  // k of this chunk within the group
      const bool ok = okP[b] && kk >= 0 && kk < r.klen;
      dma16(ok ? (const void*)(srcP[b] + k0) : (const void*)kZeroRow, lds_addr(&sP[s][(wv * CPW_P + b) * 1024]));
    }
#pragma unroll
    for (int b = 0; b < CPW_Q; ++b) {
      const int kk = k0 + chQ[b] - r.ks;
      const bool ok = kk >= 0 && kk < r.klen;
      dma16(ok ? (const void*)(srcQ[b] + k0) : (const void*)kZeroRow, lds_addr(&sQ[s][(wv * CPW_Q + b) * 1024]));
    }
    if (MX) {
      if (kRowGrouped) {
        dma4(okS ? (const void*)(srcS + kt * 4) : (const void*)kUnitScales, lds_addr(&sS[s][wv * 256]));
      } else if (wv < NW / 4) {
        const int kk = (4 * kt + kbS) * kMxBlock - r.ks;
        const bool ok = kk >= 0 && kk < r.klen;
        dma16(ok ? (const void*)(srcS + 4 * kt * kstrideS) : (const void*)kUnitScales, lds_addr(&sS[s][wv * 1024]));
      }
    }
  };
  // the copy cursor: tile ct_i, its stage ik; stage g goes to LDS buffer g % NS.
  // Tiles without k-steps (dW of an expert without tokens) have no stages.
  int ct_i = lb, ik = 0, gi = 0, gc = 0;
  TileRef ir{};
  auto seek = [&](int t0) {
    for (ct_i = t0; ct_i < total_tiles; ct_i += G) {
      ir = decode(ct_i);
      if (ir.nk > 0) {
        setup(ir);
        break;
      }
    }
    ik = 0;
  };
  auto issue_next = [&]() {
    issue(ir, ik, gi % NS);
    ++gi;
    if (++ik == ir.nk) seek(ct_i + G);
  };
  seek(lb);
#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (ct_i < total_tiles) issue_next();

  for (int t = lb; t < total_tiles; t += G) {
    const TileRef cur = decode(t);
    const int e = cur.e;
    const int64_t e64 = e;
    const int seg1 = cur.seg1, mt = cur.mt, nt = cur.nt, nk = cur.nk;
    const int row0 = cur.seg0 + mt * BM;

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int ml = lane & 15, nql = (lane >> 4) * 4, g4 = lane >> 4;
    auto compute = [&](int s) {
      int scp[TM], scq[TN];
      if (MX) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = wm * WM + i * 16 + ml;
          scp[i] = sS[s][kRowGrouped ? m * 4 + g4 : g4 * BM + m];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = wn * WN + j * 16 + ml;
          scq[j] = sS[s][kRowGrouped ? 4 * BM + n * 4 + g4 : 4 * BM + g4 * BN + n];
        }
      }
      v8i_t af[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = wm * WM + i * 16 + ml;
        const uint4 a0 = *(const uint4*)(&sP[s][rm_off(m, g4)]);
        const uint4 a1 = *(const uint4*)(&sP[s][rm_off(m, 4 + g4)]);
        af[i] = v8i_t{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
      }
      auto load_b = [&](int j) {
        const int n = wn * WN + j * 16 + ml;
        const uint4 b0 = *(const uint4*)(&sQ[s][rm_off(n, g4)]);
        const uint4 b1 = *(const uint4*)(&sQ[s][rm_off(n, 4 + g4)]);
        return v8i_t{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      };
      if constexpr (kPrefetchB) {
        // each B fragment is read from LDS one block ahead of its MFMAs, which the
        // compiler's own schedule waits for right before them; same MFMAs in the
        // same order (bit-identical)
        v8i_t bq[2];
        bq[0] = load_b(0);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (j + 1 < TN) bq[(j + 1) & 1] = load_b(j + 1);
#pragma unroll
          for (int i = 0; i < TM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bq[j & 1], af[i], acc[i][j], 0, 0, 0,
                                                                         MX ? scq[j] : 127, 0, MX ? scp[i] : 127);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const v8i_t bq = load_b(j);
#pragma unroll
          for (int i = 0; i < TM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bq, af[i], acc[i][j], 0, 0, 0,
                                                                         MX ? scq[j] : 127, 0, MX ? scp[i] : 127);
        }
      }
    };

    // dx = dg.w1 + du.w3: the w1 half (k < H) is scaled, rounded and parked in
    // the output rows, then added (in bf16) to the scaled w3 half at the end.
    auto park_dx_half = [&]() {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (r < seg1) {
            const int n = nt * BN + wn * WN + j * 16 + nql;
            float v[4];
            if (MX) {
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = acc[i][j][q];
            } else {
              const float sp = p.sp[(int64_t)r * 2];
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = (acc[i][j][q] * sp) * p.sq[e64 * 2 * D + n + q];
            }
            *(uint2*)(p.o0 + (int64_t)r * D + n) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
          }
          acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
    };
    const int kt_half = (MODE == kDx) ? H / 128 : -1;

    for (int kt = 0; kt < nk; ++kt) {
      // stage gc has landed in every wave once at most the one stage issued after it
      // is outstanding (stores of an epilogue or of the dx park only add to the
      // count); the barrier also retires every wave's reads of the buffer refilled next
      if (NS == 3 && gi - gc >= 2) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(CPW) : "memory");
      else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (ct_i < total_tiles) issue_next();
      if (MODE == kDx && kt == kt_half) park_dx_half();
      compute(gc % NS);
      ++gc;
    }
    // ---- epilogues: lane holds C[m = .. + ml][n = .. + nql + 0..3]; pairs of
    // 16-column blocks are stored as 64-byte row pieces (span64) at column
    // 32 jp + 8 (lane / 16) of the wave's span ----
    const int g8 = 8 * g4;
    // rowwise fp8, dgu and dW: the row scales of the wave's rows and the column
    // scales of its columns are loaded before the first store (a load issued after a
    // store, which may alias it, waits behind it: one round trip per tile instead of
    // one per scale; dW 2.51 -> 2.07 ms, dw2 1.28 -> 1.02 ms at 32768 Kimi tokens).
    // Rows past the segment read the segment's last row. The other epilogues keep
    // their loads in the loop: hoisted, their 32 more live registers cost the main
    // loop 5-12 %.
    constexpr bool kHoist = !MX && (MODE == kDgu || MODE >= kDw13);
    float spr[TM];
    float4 sqc[TN];
    if constexpr (kHoist) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = nt * BN + wn * WN + j * 16 + nql;
        sqc[j] = *(const float4*)((MODE == kDgu ? p.sq + e64 * H : p.sq + e64 * Ntot) + n);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (kRowGrouped) spr[i] = p.sp[min(row0 + wm * WM + i * 16 + ml, seg1 - 1)];
        else spr[i] = p.sp[e64 * Mfix + mt * BM + wm * WM + i * 16 + ml];
      }
    }
    if (MODE == kGateUp) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
          const float sx = MX ? 1.f : p.sp[r];
#pragma unroll
          for (int jp = 0; jp < TN / 4; ++jp) {
            uint2 pg[2], pu[2], ph[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int jj = 2 * jp + h2;
              const int hc = nt * (BN / 2) + wn * (WN / 2) + jj * 16 + nql;
              float gv[4], uv[4], hv[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                gv[q] = round_bf(MX ? acc[i][2 * jj][q] : (acc[i][2 * jj][q] * sx) * p.sq[e64 * H + hc + q]);
                uv[q] = round_bf(MX ? acc[i][2 * jj + 1][q] : (acc[i][2 * jj + 1][q] * sx) * p.sq2[e64 * H + hc + q]);
                // the division: the reciprocal form, chosen per four columns, measured
                // slower in this epilogue (fp8 1.67 -> 1.69 ms, MX 1.73 -> 1.74 ms)
                hv[q] = round_bf(silu_sig<false>(gv[q], silu_den(gv[q])).silu) * uv[q];
              }
              pg[h2] = pack4(gv);
              pu[h2] = pack4(uv);
              ph[h2] = pack4(hv);
            }
            const int64_t off = (int64_t)r * H + nt * (BN / 2) + wn * (WN / 2) + jp * 32 + g8;
            const uint4 sg = span64(pg[0], pg[1], lane), su = span64(pu[0], pu[1], lane),
                        sh = span64(ph[0], ph[1], lane);
            *(uint4*)(p.o0 + off) = sg;
            *(uint4*)(p.o1 + off) = su;
            *(uint4*)(p.o2 + off) = sh;
          }
        }
      }
    } else if (MODE == kDown || MODE == kDx) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
          const float sp = MX ? 1.f : ((MODE == kDx) ? p.sp[(int64_t)r * 2 + 1] : p.sp[r]);
          // MXFP8 dx: the parked w1 half of the row, read back before the row's stores
          // (rowwise fp8 reads it piece by piece: its scale loads already hold the
          // registers this would take)
          constexpr bool kBatchPark = MODE == kDx && MX;
          uint2 pws[kBatchPark ? TN : 1];
          if constexpr (kBatchPark) {
#pragma unroll
            for (int j = 0; j < TN; ++j) pws[j] = *(const uint2*)(p.o0 + (int64_t)r * D + nt * BN + wn * WN + j * 16 + nql);
          }
#pragma unroll
          for (int jp = 0; jp < TN / 2; ++jp) {
            uint2 pv[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int j = 2 * jp + h2;
              const int n = nt * BN + wn * WN + j * 16 + nql;
              float v[4];
              if (MX) {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = acc[i][j][q];
              } else {
                const float* sq = (MODE == kDx) ? p.sq + e64 * 2 * D + D + n : p.sq + e64 * D + n;
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = (acc[i][j][q] * sp) * sq[q];
              }
              if constexpr (MODE == kDx) {
                uint2 pw;
                if constexpr (kBatchPark) pw = pws[j];
                else pw = *(const uint2*)(p.o0 + (int64_t)r * D + n);
                v[0] = bf_lo(pw.x) + round_bf(v[0]);
                v[1] = bf_hi(pw.x) + round_bf(v[1]);
                v[2] = bf_lo(pw.y) + round_bf(v[2]);
                v[3] = bf_hi(pw.y) + round_bf(v[3]);
              }
              pv[h2] = pack4(v);
            }
            const uint4 sv = span64(pv[0], pv[1], lane);
            *(uint4*)(p.o0 + (int64_t)r * D + nt * BN + wn * WN + jp * 32 + g8) = sv;
          }
        }
      }
    } else if (MODE == kDgu) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
          const float sp = MX ? 1.f : spr[i];
          // the g and u pieces of half the row's columns at a time, loaded before their
          // stores (registers for all of them at once would spill)
          uint2 gws[TN / 2], uws[TN / 2];
#pragma unroll
          for (int jp = 0; jp < TN / 2; ++jp) {
            if (jp % (TN / 4) == 0) {
#pragma unroll
              for (int jj = 0; jj < TN / 2; ++jj) {
                const int64_t off = (int64_t)r * H + nt * BN + wn * WN + (2 * jp + jj) * 16 + nql;
                gws[jj] = *(const uint2*)(p.g + off);
                uws[jj] = *(const uint2*)(p.u + off);
              }
            }
            uint2 pdg[2], pdu[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int j = 2 * jp + h2;
              const uint2 gw = gws[j % (TN / 2)], uw = uws[j % (TN / 2)];
              const float gv[4] = {bf_lo(gw.x), bf_hi(gw.x), bf_lo(gw.y), bf_hi(gw.y)};
              const float uv[4] = {bf_lo(uw.x), bf_hi(uw.x), bf_lo(uw.y), bf_hi(uw.y)};
              float dg[4], du[4];
              float sq4[4] = {1.f, 1.f, 1.f, 1.f};
              if constexpr (!MX) {
                sq4[0] = sqc[j].x; sq4[1] = sqc[j].y; sq4[2] = sqc[j].z; sq4[3] = sqc[j].w;
              }
              if constexpr (MX) {
                // silu and sigmoid in the reciprocal form where a pair of columns lies
                // in its range for every lane (MX dgu 1.29 -> 1.22 ms at 32K Kimi tokens)
#pragma unroll
                for (int q = 0; q < 4; q += 2) {
                  const float d0 = silu_den(gv[q]), d1 = silu_den(gv[q + 1]);
                  SiluSig f[2];
                  if (silu_fast_wave(fminf(gv[q], gv[q + 1]), fmaxf(gv[q], gv[q + 1]))) {
                    f[0] = silu_sig<true>(gv[q], d0);
                    f[1] = silu_sig<true>(gv[q + 1], d1);
                  } else {
                    f[0] = silu_sig<false>(gv[q], d0);
                    f[1] = silu_sig<false>(gv[q + 1], d1);
                  }
#pragma unroll
                  for (int t = 0; t < 2; ++t) {
                    const float dh = round_bf(acc[i][j][q + t]);
                    const float sl = round_bf(f[t].silu);
                    const float dsl = round_bf(dh * uv[q + t]);
                    du[q + t] = dh * sl;
                    const float sg = f[t].sig;
                    dg[q + t] = dsl * sg * (1.0f + gv[q + t] * (1.0f - sg));
                  }
                }
              } else {
                // the division itself: the rowwise variant holds its scales across the
                // epilogue, and the reciprocal form's branch spilled it or, per four
                // columns, made it slower (1.33 -> 1.38 ms)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  const float dh = round_bf((acc[i][j][q] * sp) * sq4[q]);
                  const float sl = round_bf(gv[q] / (1.0f + expf(-gv[q])));
                  const float dsl = round_bf(dh * uv[q]);
                  du[q] = dh * sl;
                  const float sg = 1.0f / (1.0f + expf(-gv[q]));
                  dg[q] = dsl * sg * (1.0f + gv[q] * (1.0f - sg));
                }
              }
              pdg[h2] = pack4(dg);
              pdu[h2] = pack4(du);
            }
            const int64_t o2 = (int64_t)r * (2 * H) + nt * BN + wn * WN + jp * 32 + g8;
            // rowwise: the crossbar exchange (the lane swaps measured 1.33 -> 1.36 ms here)
            const uint4 sdg = MX ? span64(pdg[0], pdg[1], lane) : span64_lds(pdg[0], pdg[1], lane);
            const uint4 sdu = MX ? span64(pdu[0], pdu[1], lane) : span64_lds(pdu[0], pdu[1], lane);
            *(uint4*)(p.o0 + o2) = sdg;
            *(uint4*)(p.o0 + o2 + H) = sdu;
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = mt * BM + wm * WM + i * 16 + ml;
        // an expert without tokens gets zero gradients (its scales are never written)
        const float sp = MX ? 1.f : spr[i];
        uint16_t* rowp;
        if (MODE == kDw13)
          rowp = (m < H) ? p.o0 + (e64 * H + m) * (int64_t)D : p.o1 + (e64 * H + (m - H)) * (int64_t)D;
        else
          rowp = p.o0 + (e64 * D + m) * (int64_t)H;
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          uint2 pv[2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int j = 2 * jp + h2;
            const int n = nt * BN + wn * WN + j * 16 + nql;
            float v[4];
            float sq4[4] = {1.f, 1.f, 1.f, 1.f};
            if constexpr (!MX) {
              sq4[0] = sqc[j].x; sq4[1] = sqc[j].y; sq4[2] = sqc[j].z; sq4[3] = sqc[j].w;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = (nk > 0) ? (MX ? acc[i][j][q] : (acc[i][j][q] * sp) * sq4[q]) : 0.f;
            pv[h2] = pack4(v);
          }
          *(uint4*)(rowp + nt * BN + wn * WN + jp * 32 + g8) = span64(pv[0], pv[1], lane);
        }
      }
    }
  }
}

static int g_cus[64];
static int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!g_cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

template <int MODE, int NW, int WGM, int TM, int TN, int NS, int OCC, bool MX>
static void launch_cfg(const Params& p, hipStream_t stream) {
  constexpr int BM = WGM * TM * 16, BN = (NW / WGM) * TN * 16;
  int64_t max_tiles;
  if (MODE == kGateUp) max_tiles = (p.R / BM + p.E) * (2 * p.H / BN);
  else if (MODE == kDown || MODE == kDx) max_tiles = (p.R / BM + p.E) * (p.D / BN);
  else if (MODE == kDgu) max_tiles = (p.R / BM + p.E) * (p.H / BN);
  else if (MODE == kDw13) max_tiles = (int64_t)p.E * (2 * p.H / BM) * (p.D / BN);
  else max_tiles = (int64_t)p.E * (p.D / BM) * (p.H / BN);
  int64_t g = (int64_t)cu_count() * OCC;
  if (g > max_tiles) g = max_tiles;
  if (g >= 8) g -= g % 8;
  if (g < 1) g = 1;
  hipLaunchKernelGGL((fp8_gemm_kernel<MODE, NW, WGM, TM, TN, NS, OCC, MX>), dim3((int)g), dim3(NW * 64), 0, stream, p);
}

// Tiles (measured at the Kimi shape, 32768 tokens): 256 x 256 outputs of eight
// 64 x 128 wave tiles, two 64 KB stages, one workgroup per CU -- half the copy
// bytes per MFMA of 128 x 128 tiles of four waves (six GEMMs: fp8 11.4 -> 9.6 ms,
// MXFP8 10.9 -> 9.0 ms). D and H are multiples of 256 (check_shape), so every
// n-tile and dW m-tile is whole.
template <int MODE, bool MX = false>
static void launch(const Params& p, hipStream_t stream) {
  launch_cfg<MODE, 8, 4, 4, 8, 2, 1, MX>(p, stream);
}

static int check_shape(int64_t R, int E, int D, int H) {
  if (R < 0 || E < 1 || E > kMaxE || D < 256 || H < 256) return kErrInvalidArgument;
  if (D % 256 || H % 256) return kErrUnsupportedShape;
  if (R >= (int64_t)INT32_MAX / 2) return kErrUnsupportedShape;
  return kOk;
}

}  // namespace fp8
}  // namespace moe

using namespace moe;
using namespace moe::fp8;

MOE_API int64_t moe_fp8_padded_rows(int64_t n_rows, int32_t n_experts) {
  return n_rows + (int64_t)n_experts * (kPad - 1);
}

MOE_API int moe_fp8_quant_rows(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q, float* scale,
                               hipStream_t stream) {
  if (rows < 0 || cols < 8 || cols % 8) return kErrInvalidArgument;
  if (rows == 0) return kOk;
  if (!x || !q || !scale) return kErrInvalidArgument;
  int64_t g = (rows + 3) / 4;
  if (g > 16384) g = 16384;
  const int chunks = cols / 8;
  if (chunks <= 64 * 2)
    hipLaunchKernelGGL(quant_rows_kernel<2>, dim3((int)g), dim3(256), 0, stream, x, rows, cols, q, scale);
  else if (chunks <= 64 * 4)
    hipLaunchKernelGGL(quant_rows_kernel<4>, dim3((int)g), dim3(256), 0, stream, x, rows, cols, q, scale);
  else if (chunks <= 64 * 8)
    hipLaunchKernelGGL(quant_rows_kernel<8>, dim3((int)g), dim3(256), 0, stream, x, rows, cols, q, scale);
  else if (chunks <= 64 * 16)
    hipLaunchKernelGGL(quant_rows_kernel<16>, dim3((int)g), dim3(256), 0, stream, x, rows, cols, q, scale);
  else
    hipLaunchKernelGGL(quant_rows_kernel<0>, dim3((int)g), dim3(256), 0, stream, x, rows, cols, q, scale);
  return launch_status();
}

static int quant_cols_t(const uint16_t* x, const float* col_amax, int32_t n_experts, int32_t a, int32_t b,
                        uint8_t* q, int64_t q_expert_stride, int64_t q_row_stride, float* scale,
                        int64_t scale_expert_stride, hipStream_t stream) {
  if (n_experts < 1 || a < 16 || a % 16 || b < 64 || b % 64) return kErrInvalidArgument;
  if (q_row_stride < a || q_row_stride % 16 || q_expert_stride < (int64_t)(b - 1) * q_row_stride + a ||
      scale_expert_stride < b)
    return kErrInvalidArgument;
  if (!x || !q || !scale) return kErrInvalidArgument;
  if (b % 128 == 0)
    hipLaunchKernelGGL(quant_cols_t_kernel<128>, dim3(n_experts * (b / 128)), dim3(512), 0, stream, x, a, b, q,
                       q_expert_stride, q_row_stride, scale, scale_expert_stride, col_amax);
  else
    hipLaunchKernelGGL(quant_cols_t_kernel<64>, dim3(n_experts * (b / 64)), dim3(256), 0, stream, x, a, b, q,
                       q_expert_stride, q_row_stride, scale, scale_expert_stride, col_amax);
  return launch_status();
}

MOE_API int moe_fp8_quant_cols_t(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q,
                                 int64_t q_expert_stride, int64_t q_row_stride, float* scale,
                                 int64_t scale_expert_stride, hipStream_t stream) {
  return quant_cols_t(x, nullptr, n_experts, a, b, q, q_expert_stride, q_row_stride, scale, scale_expert_stride,
                      stream);
}

MOE_API int moe_fp8_quant_cols_t_amax(const uint16_t* x, const float* col_amax, int32_t n_experts, int32_t a,
                                      int32_t b, uint8_t* q, int64_t q_expert_stride, int64_t q_row_stride,
                                      float* scale, int64_t scale_expert_stride, hipStream_t stream) {
  if (!col_amax) return kErrInvalidArgument;
  return quant_cols_t(x, col_amax, n_experts, a, b, q, q_expert_stride, q_row_stride, scale, scale_expert_stride,
                      stream);
}

MOE_API int moe_fp8_quant_rows_colamax(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q,
                                       float* scale, float* col_amax, hipStream_t stream) {
  if (n_experts < 1 || a < 1 || b < 8 || b % 8 || b > 8192) return kErrInvalidArgument;
  if (!x || !q || !scale || !col_amax) return kErrInvalidArgument;
  // E x S blocks, S row slices per expert: sixteen blocks per CU (at the Kimi
  // weights 0.37 ms against 0.38-0.44 ms for two to eight per CU; a slice's
  // atomics are one per column)
  int s = (16 * cu_count() + n_experts - 1) / n_experts;
  if (s > a) s = a;
  const int rb = (a + s - 1) / s;
  const dim3 grid((a + rb - 1) / rb, n_experts), block(256);
  uint32_t* cm = (uint32_t*)col_amax;
  const int chunks = b / 8;
  if (chunks <= 64 * 2)
    hipLaunchKernelGGL(quant_rows_colamax_kernel<2>, grid, block, 0, stream, x, a, b, rb, q, scale, cm);
  else if (chunks <= 64 * 4)
    hipLaunchKernelGGL(quant_rows_colamax_kernel<4>, grid, block, 0, stream, x, a, b, rb, q, scale, cm);
  else if (chunks <= 64 * 5)
    hipLaunchKernelGGL(quant_rows_colamax_kernel<5>, grid, block, 0, stream, x, a, b, rb, q, scale, cm);
  else if (chunks <= 64 * 8)
    hipLaunchKernelGGL(quant_rows_colamax_kernel<8>, grid, block, 0, stream, x, a, b, rb, q, scale, cm);
  else
    hipLaunchKernelGGL(quant_rows_colamax_kernel<16>, grid, block, 0, stream, x, a, b, rb, q, scale, cm);
  return launch_status();
}

static int quant_tokens_t(const uint16_t* x, const float* group_amax, const int64_t* counts, int64_t n_rows,
                          int32_t n_experts, int32_t cols, int64_t padded_rows, uint8_t* q, float* scale,
                          hipStream_t stream, RowGather gather = RowGather{}) {
  if (n_rows < 0 || n_experts < 1 || n_experts > kMaxE || cols < 64 || cols % 64) return kErrInvalidArgument;
  if (padded_rows < moe_fp8_padded_rows(n_rows, n_experts) || padded_rows % kPad) return kErrWorkspace;
  if (!x || !counts || !q || !scale) return kErrInvalidArgument;
  const bool g = gather.idx != nullptr;
  using kernel_t = void (*)(const uint16_t*, const int64_t*, int64_t, int, int, int64_t, uint8_t*, float*,
                            const float*, RowGather);
  const kernel_t k128 = g ? quant_tokens_t_kernel<128, true> : quant_tokens_t_kernel<128, false>;
  const kernel_t k64 = g ? quant_tokens_t_kernel<64, true> : quant_tokens_t_kernel<64, false>;
  if (cols % 128 == 0)
    hipLaunchKernelGGL(k128, dim3(n_experts * (cols / 128)), dim3(512), 0, stream, x, counts, n_rows, n_experts, cols,
                       padded_rows, q, scale, group_amax, gather);
  else
    hipLaunchKernelGGL(k64, dim3(n_experts * (cols / 64)), dim3(256), 0, stream, x, counts, n_rows, n_experts, cols,
                       padded_rows, q, scale, group_amax, gather);
  return launch_status();
}

MOE_API int moe_fp8_quant_tokens_t(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                   int32_t cols, int64_t padded_rows, uint8_t* q, float* scale,
                                   hipStream_t stream) {
  return quant_tokens_t(x, nullptr, counts, n_rows, n_experts, cols, padded_rows, q, scale, stream);
}

MOE_API int moe_fp8_quant_tokens_t_amax(const uint16_t* x, const float* group_amax, const int64_t* counts,
                                        int64_t n_rows, int32_t n_experts, int32_t cols, int64_t padded_rows,
                                        uint8_t* q, float* scale, hipStream_t stream) {
  if (!group_amax) return kErrInvalidArgument;
  return quant_tokens_t(x, group_amax, counts, n_rows, n_experts, cols, padded_rows, q, scale, stream);
}

template <int P, bool G>
static void launch_rows_groupamax(int chunks, dim3 grid, hipStream_t stream, const uint16_t* x, const int64_t* counts,
                                  int64_t rows, int e, int cols, int rb, uint8_t* q, float* scale, uint32_t* gam,
                                  RowGather gather) {
  if (chunks <= 64 * 2)
    hipLaunchKernelGGL((quant_rows_groupamax_kernel<2, P, G>), grid, dim3(256), 0, stream, x, counts, rows, e, cols,
                       rb, q, scale, gam, gather);
  else if (chunks <= 64 * 4)
    hipLaunchKernelGGL((quant_rows_groupamax_kernel<4, P, G>), grid, dim3(256), 0, stream, x, counts, rows, e, cols,
                       rb, q, scale, gam, gather);
  else if (chunks <= 64 * 5)
    hipLaunchKernelGGL((quant_rows_groupamax_kernel<5, P, G>), grid, dim3(256), 0, stream, x, counts, rows, e, cols,
                       rb, q, scale, gam, gather);
  else if (chunks <= 64 * 8)
    hipLaunchKernelGGL((quant_rows_groupamax_kernel<8, P, G>), grid, dim3(256), 0, stream, x, counts, rows, e, cols,
                       rb, q, scale, gam, gather);
  else
    hipLaunchKernelGGL((quant_rows_groupamax_kernel<16, P, G>), grid, dim3(256), 0, stream, x, counts, rows, e, cols,
                       rb, q, scale, gam, gather);
}

static int rows_groupamax(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                          int32_t cols, int32_t pieces, uint8_t* q, float* scale, float* group_amax,
                          hipStream_t stream, RowGather gather = RowGather{}) {
  if (n_rows < 0 || n_experts < 1 || n_experts > kMaxE || (pieces != 1 && pieces != 2)) return kErrInvalidArgument;
  if (cols < 8 * pieces || cols % (8 * pieces) || cols > 8192) return kErrInvalidArgument;
  if (n_rows >= (int64_t)INT32_MAX / 2) return kErrUnsupportedShape;
  if (n_rows == 0) return kOk;
  if (!x || !counts || !q || !scale || !group_amax) return kErrInvalidArgument;
  // blocks of RB consecutive rows, sixteen per CU (a block's atomics are one per
  // column for each group it leaves)
  const int64_t want = 16 * (int64_t)cu_count();
  int64_t rb = (n_rows + want - 1) / want;
  if (rb < 16) rb = 16;
  const dim3 grid((unsigned)((n_rows + rb - 1) / rb));
  uint32_t* gam = (uint32_t*)group_amax;
  if (gather.idx)
    launch_rows_groupamax<1, true>(cols / 8, grid, stream, x, counts, n_rows, n_experts, cols, (int)rb, q, scale, gam,
                                   gather);
  else if (pieces == 1)
    launch_rows_groupamax<1, false>(cols / 8, grid, stream, x, counts, n_rows, n_experts, cols, (int)rb, q, scale,
                                    gam, gather);
  else
    launch_rows_groupamax<2, false>(cols / 8, grid, stream, x, counts, n_rows, n_experts, cols, (int)rb, q, scale,
                                    gam, gather);
  return launch_status();
}

MOE_API int moe_fp8_quant_rows_groupamax(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                         int32_t cols, int32_t pieces, uint8_t* q, float* scale, float* group_amax,
                                         hipStream_t stream) {
  return rows_groupamax(x, counts, n_rows, n_experts, cols, pieces, q, scale, group_amax, stream);
}

static int row_gather(RowGather& g, const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                      const float* row_scale, int32_t cols) {
  if (n_src < 1 || !token_idx || reinterpret_cast<uintptr_t>(src) % 16) return kErrInvalidArgument;
  g.src = src;
  g.idx = token_idx;
  g.scale = row_scale;
  g.ld = cols;
  g.n_src = n_src;
  return kOk;
}

MOE_API int moe_fp8_quant_rows_groupamax_gather(const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                                                const float* row_scale, const int64_t* counts, int64_t n_rows,
                                                int32_t n_experts, int32_t cols, uint8_t* q, float* scale,
                                                float* group_amax, hipStream_t stream) {
  RowGather g;
  const int st = row_gather(g, src, n_src, token_idx, row_scale, cols);
  if (st) return st;
  return rows_groupamax(src, counts, n_rows, n_experts, cols, 1, q, scale, group_amax, stream, g);
}

MOE_API int moe_fp8_quant_tokens_t_amax_gather(const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                                               const float* row_scale, const float* group_amax,
                                               const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                               int32_t cols, int64_t padded_rows, uint8_t* q, float* scale,
                                               hipStream_t stream) {
  if (!group_amax) return kErrInvalidArgument;
  RowGather g;
  const int st = row_gather(g, src, n_src, token_idx, row_scale, cols);
  if (st) return st;
  return quant_tokens_t(src, group_amax, counts, n_rows, n_experts, cols, padded_rows, q, scale, stream, g);
}

static int fp8_params(Params& p, const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                      int32_t hidden) {
  const int st = check_shape(n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (!counts) return kErrInvalidArgument;
  p = Params{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.D = dim; p.H = hidden;
  return kOk;
}

MOE_API int moe_fp8_gemm_gate_up(const uint8_t* qx, const float* sx, const uint8_t* qw1, const float* sw1,
                                 const uint8_t* qw3, const float* sw3, const int64_t* counts, int64_t n_rows,
                                 int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* g, uint16_t* u,
                                 uint16_t* h, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qx || !sx || !qw1 || !sw1 || !qw3 || !sw3 || !g || !u || !h) return kErrInvalidArgument;
  p.qp = qx; p.sp = sx; p.qq = qw1; p.sq = sw1; p.qq2 = qw3; p.sq2 = sw3; p.o0 = g; p.o1 = u; p.o2 = h;
  launch<kGateUp>(p, stream);
  return launch_status();
}

MOE_API int moe_fp8_gemm_down(const uint8_t* qh, const float* sh, const uint8_t* qw2, const float* sw2,
                              const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                              int32_t hidden, uint16_t* y, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qh || !sh || !qw2 || !sw2 || !y) return kErrInvalidArgument;
  p.qp = qh; p.sp = sh; p.qq = qw2; p.sq = sw2; p.o0 = y;
  launch<kDown>(p, stream);
  return launch_status();
}

MOE_API int moe_fp8_gemm_bwd_dgu(const uint8_t* qdy, const float* sdy, const uint8_t* qw2t, const float* sw2t,
                                 const uint16_t* g, const uint16_t* u, const int64_t* counts, int64_t n_rows,
                                 int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dgu,
                                 hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qdy || !sdy || !qw2t || !sw2t || !g || !u || !dgu) return kErrInvalidArgument;
  p.qp = qdy; p.sp = sdy; p.qq = qw2t; p.sq = sw2t; p.g = g; p.u = u; p.o0 = dgu;
  launch<kDgu>(p, stream);
  return launch_status();
}

MOE_API int moe_fp8_gemm_bwd_dx(const uint8_t* qdgu, const float* sdgu, const uint8_t* qw13t, const float* sw13t,
                                const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                int32_t hidden, uint16_t* dx, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qdgu || !sdgu || !qw13t || !sw13t || !dx) return kErrInvalidArgument;
  p.qp = qdgu; p.sp = sdgu; p.qq = qw13t; p.sq = sw13t; p.o0 = dx;
  launch<kDx>(p, stream);
  return launch_status();
}

MOE_API int moe_fp8_gemm_bwd_dw13(const uint8_t* qdgut, const float* sdgut, const uint8_t* qxt, const float* sxt,
                                  const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                                  int32_t dim, int32_t hidden, uint16_t* dw1, uint16_t* dw3, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (padded_rows < moe_fp8_padded_rows(n_rows, n_experts) || padded_rows % kPad) return kErrWorkspace;
  if (!dw1 || !dw3 || (n_rows > 0 && (!qdgut || !sdgut || !qxt || !sxt))) return kErrInvalidArgument;
  p.Rpad = padded_rows; p.qp = qdgut; p.sp = sdgut; p.qq = qxt; p.sq = sxt; p.o0 = dw1; p.o1 = dw3;
  launch<kDw13>(p, stream);
  return launch_status();
}

MOE_API int moe_fp8_gemm_bwd_dw2(const uint8_t* qdyt, const float* sdyt, const uint8_t* qht, const float* sht,
                                 const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                                 int32_t dim, int32_t hidden, uint16_t* dw2, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (padded_rows < moe_fp8_padded_rows(n_rows, n_experts) || padded_rows % kPad) return kErrWorkspace;
  if (!dw2 || (n_rows > 0 && (!qdyt || !sdyt || !qht || !sht))) return kErrInvalidArgument;
  p.Rpad = padded_rows; p.qp = qdyt; p.sp = sdyt; p.qq = qht; p.sq = sht; p.o0 = dw2;
  launch<kDw2>(p, stream);
  return launch_status();
}

// ---------------------------------------------------------------------------
// MXFP8 entry points (e8m0 scales as uint8 bytes)
// ---------------------------------------------------------------------------

MOE_API int64_t moe_mxfp8_padded_rows(int64_t n_rows, int32_t n_experts) {
  const int64_t n = n_rows + (int64_t)n_experts * (kMxPad - 1);
  return (n + kMxPad - 1) / kMxPad * kMxPad;
}

MOE_API int moe_mxfp8_quant_rows(const uint16_t* x, int64_t rows, int32_t cols, uint8_t* q, uint8_t* scale,
                                 hipStream_t stream) {
  if (rows < 0 || cols < kMxBlock || cols % kMxBlock) return kErrInvalidArgument;
  if (rows == 0) return kOk;
  if (!x || !q || !scale) return kErrInvalidArgument;
  const int64_t chunks = rows * (cols / 8);
  int64_t g = (chunks + 4 * 256 - 1) / (4 * 256);
  if (g > 32768) g = 32768;
  hipLaunchKernelGGL(mx_quant_rows_kernel, dim3((int)g), dim3(256), 0, stream, (const uint4*)x, chunks, (uint2*)q,
                     scale);
  return launch_status();
}

MOE_API int moe_mxfp8_quant_cols_t(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q,
                                   int64_t q_expert_stride, int64_t q_row_stride, uint8_t* scale,
                                   int64_t scale_expert_stride, int64_t scale_row_stride, hipStream_t stream) {
  if (n_experts < 1 || a < kMxBlock || a % kMxBlock || b < 64 || b % 64) return kErrInvalidArgument;
  if (q_row_stride < a || q_row_stride % 16 || q_expert_stride < (int64_t)(b - 1) * q_row_stride + a)
    return kErrInvalidArgument;
  if (scale_row_stride < a / kMxBlock || scale_expert_stride < (int64_t)(b - 1) * scale_row_stride + a / kMxBlock)
    return kErrInvalidArgument;
  if (!x || !q || !scale) return kErrInvalidArgument;
  if (b % 128 == 0)
    hipLaunchKernelGGL(mx_quant_cols_t_kernel<128>, dim3(n_experts * (b / 128)), dim3(512), 0, stream, x, a, b, q,
                       q_expert_stride, q_row_stride, scale, scale_expert_stride, scale_row_stride);
  else
    hipLaunchKernelGGL(mx_quant_cols_t_kernel<64>, dim3(n_experts * (b / 64)), dim3(256), 0, stream, x, a, b, q,
                       q_expert_stride, q_row_stride, scale, scale_expert_stride, scale_row_stride);
  return launch_status();
}

MOE_API int moe_mxfp8_quant_tokens_t(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                     int32_t cols, int64_t padded_rows, uint8_t* q, uint8_t* scale,
                                     hipStream_t stream) {
  if (n_rows < 0 || n_experts < 1 || n_experts > kMaxE || cols < 64 || cols % 64) return kErrInvalidArgument;
  if (padded_rows < moe_mxfp8_padded_rows(n_rows, n_experts) || padded_rows % kMxPad) return kErrWorkspace;
  if (!x || !counts || !q || !scale) return kErrInvalidArgument;
  if (cols % 128 == 0)
    hipLaunchKernelGGL((mx_quant_tokens_t_kernel<false, 128>), dim3(n_experts * (cols / 128)), dim3(512), 0, stream, x,
                       counts, n_rows, n_experts, cols, padded_rows, q, scale, (uint8_t*)nullptr, (uint8_t*)nullptr,
                       RowGather{});
  else
    hipLaunchKernelGGL((mx_quant_tokens_t_kernel<false, 64>), dim3(n_experts * (cols / 64)), dim3(256), 0, stream, x,
                       counts, n_rows, n_experts, cols, padded_rows, q, scale, (uint8_t*)nullptr, (uint8_t*)nullptr,
                       RowGather{});
  return launch_status();
}

MOE_API int moe_mxfp8_quant_dual_cols(const uint16_t* x, int32_t n_experts, int32_t a, int32_t b, uint8_t* q_rows,
                                      uint8_t* scale_rows, uint8_t* q, int64_t q_expert_stride, int64_t q_row_stride,
                                      uint8_t* scale, int64_t scale_expert_stride, int64_t scale_row_stride,
                                      hipStream_t stream) {
  if (n_experts < 1 || a < kMxBlock || a % kMxBlock || b < 64 || b % 64) return kErrInvalidArgument;
  if (q_row_stride < a || q_row_stride % 16 || q_expert_stride < (int64_t)(b - 1) * q_row_stride + a)
    return kErrInvalidArgument;
  if (scale_row_stride < a / kMxBlock || scale_expert_stride < (int64_t)(b - 1) * scale_row_stride + a / kMxBlock)
    return kErrInvalidArgument;
  if (!x || !q || !scale || !q_rows || !scale_rows) return kErrInvalidArgument;
  if (b % 128 == 0)
    hipLaunchKernelGGL(mx_dual_cols_kernel<128>, dim3(n_experts * (b / 128)), dim3(512), 0, stream, x, a, b, q,
                       q_expert_stride, q_row_stride, scale, scale_expert_stride, scale_row_stride, q_rows, scale_rows);
  else
    hipLaunchKernelGGL(mx_dual_cols_kernel<64>, dim3(n_experts * (b / 64)), dim3(256), 0, stream, x, a, b, q,
                       q_expert_stride, q_row_stride, scale, scale_expert_stride, scale_row_stride, q_rows, scale_rows);
  return launch_status();
}

static int mx_dual_tokens(const uint16_t* x, RowGather gather, const int64_t* counts, int64_t n_rows,
                          int32_t n_experts, int32_t cols, int64_t padded_rows, uint8_t* q_rows, uint8_t* scale_rows,
                          uint8_t* q, uint8_t* scale, hipStream_t stream) {
  if (n_rows < 0 || n_experts < 1 || n_experts > kMaxE || cols < 64 || cols % 64) return kErrInvalidArgument;
  if (padded_rows < moe_mxfp8_padded_rows(n_rows, n_experts) || padded_rows % kMxPad) return kErrWorkspace;
  if (!x || !counts || !q || !scale || !q_rows || !scale_rows) return kErrInvalidArgument;
  const bool g = gather.idx != nullptr;
  using kernel_t = void (*)(const uint16_t*, const int64_t*, int64_t, int, int, int64_t, uint8_t*, uint8_t*, uint8_t*,
                            uint8_t*, RowGather);
  const kernel_t k128 = g ? mx_quant_tokens_t_kernel<true, 128, true> : mx_quant_tokens_t_kernel<true, 128, false>;
  const kernel_t k64 = g ? mx_quant_tokens_t_kernel<true, 64, true> : mx_quant_tokens_t_kernel<true, 64, false>;
  if (cols % 128 == 0)
    hipLaunchKernelGGL(k128, dim3(n_experts * (cols / 128)), dim3(512), 0, stream, x, counts, n_rows, n_experts, cols,
                       padded_rows, q, scale, q_rows, scale_rows, gather);
  else
    hipLaunchKernelGGL(k64, dim3(n_experts * (cols / 64)), dim3(256), 0, stream, x, counts, n_rows, n_experts, cols,
                       padded_rows, q, scale, q_rows, scale_rows, gather);
  return launch_status();
}

MOE_API int moe_mxfp8_quant_dual_tokens(const uint16_t* x, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                        int32_t cols, int64_t padded_rows, uint8_t* q_rows, uint8_t* scale_rows,
                                        uint8_t* q, uint8_t* scale, hipStream_t stream) {
  return mx_dual_tokens(x, RowGather{}, counts, n_rows, n_experts, cols, padded_rows, q_rows, scale_rows, q, scale,
                        stream);
}

MOE_API int moe_mxfp8_quant_dual_tokens_gather(const uint16_t* src, int64_t n_src, const int64_t* token_idx,
                                               const float* row_scale, const int64_t* counts, int64_t n_rows,
                                               int32_t n_experts, int32_t cols, int64_t padded_rows,
                                               uint8_t* q_rows, uint8_t* scale_rows, uint8_t* q, uint8_t* scale,
                                               hipStream_t stream) {
  RowGather g;
  const int st = row_gather(g, src, n_src, token_idx, row_scale, cols);
  if (st) return st;
  return mx_dual_tokens(src, g, counts, n_rows, n_experts, cols, padded_rows, q_rows, scale_rows, q, scale, stream);
}

MOE_API int moe_mxfp8_gemm_gate_up(const uint8_t* qx, const uint8_t* sx, const uint8_t* qw1, const uint8_t* sw1,
                                   const uint8_t* qw3, const uint8_t* sw3, const int64_t* counts, int64_t n_rows,
                                   int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* g, uint16_t* u,
                                   uint16_t* h, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qx || !sx || !qw1 || !sw1 || !qw3 || !sw3 || !g || !u || !h) return kErrInvalidArgument;
  p.qp = qx; p.ep = sx; p.qq = qw1; p.eq = sw1; p.qq2 = qw3; p.eq2 = sw3; p.o0 = g; p.o1 = u; p.o2 = h;
  launch<kGateUp, true>(p, stream);
  return launch_status();
}

MOE_API int moe_mxfp8_gemm_down(const uint8_t* qh, const uint8_t* sh, const uint8_t* qw2, const uint8_t* sw2,
                                const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                int32_t hidden, uint16_t* y, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qh || !sh || !qw2 || !sw2 || !y) return kErrInvalidArgument;
  p.qp = qh; p.ep = sh; p.qq = qw2; p.eq = sw2; p.o0 = y;
  launch<kDown, true>(p, stream);
  return launch_status();
}

MOE_API int moe_mxfp8_gemm_bwd_dgu(const uint8_t* qdy, const uint8_t* sdy, const uint8_t* qw2t,
                                   const uint8_t* sw2t, const uint16_t* g, const uint16_t* u, const int64_t* counts,
                                   int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dgu,
                                   hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qdy || !sdy || !qw2t || !sw2t || !g || !u || !dgu) return kErrInvalidArgument;
  p.qp = qdy; p.ep = sdy; p.qq = qw2t; p.eq = sw2t; p.g = g; p.u = u; p.o0 = dgu;
  launch<kDgu, true>(p, stream);
  return launch_status();
}

MOE_API int moe_mxfp8_gemm_bwd_dx(const uint8_t* qdgu, const uint8_t* sdgu, const uint8_t* qw13t,
                                  const uint8_t* sw13t, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                  int32_t dim, int32_t hidden, uint16_t* dx, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!qdgu || !sdgu || !qw13t || !sw13t || !dx) return kErrInvalidArgument;
  p.qp = qdgu; p.ep = sdgu; p.qq = qw13t; p.eq = sw13t; p.o0 = dx;
  launch<kDx, true>(p, stream);
  return launch_status();
}

MOE_API int moe_mxfp8_gemm_bwd_dw13(const uint8_t* qdgut, const uint8_t* sdgut, const uint8_t* qxt,
                                    const uint8_t* sxt, const int64_t* counts, int64_t n_rows, int64_t padded_rows,
                                    int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dw1, uint16_t* dw3,
                                    hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (padded_rows < moe_mxfp8_padded_rows(n_rows, n_experts) || padded_rows % kMxPad) return kErrWorkspace;
  if (!dw1 || !dw3 || (n_rows > 0 && (!qdgut || !sdgut || !qxt || !sxt))) return kErrInvalidArgument;
  p.Rpad = padded_rows; p.qp = qdgut; p.ep = sdgut; p.qq = qxt; p.eq = sxt; p.o0 = dw1; p.o1 = dw3;
  launch<kDw13, true>(p, stream);
  return launch_status();
}

MOE_API int moe_mxfp8_gemm_bwd_dw2(const uint8_t* qdyt, const uint8_t* sdyt, const uint8_t* qht, const uint8_t* sht,
                                   const int64_t* counts, int64_t n_rows, int64_t padded_rows, int32_t n_experts,
                                   int32_t dim, int32_t hidden, uint16_t* dw2, hipStream_t stream) {
  Params p;
  int st = fp8_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (padded_rows < moe_mxfp8_padded_rows(n_rows, n_experts) || padded_rows % kMxPad) return kErrWorkspace;
  if (!dw2 || (n_rows > 0 && (!qdyt || !sdyt || !qht || !sht))) return kErrInvalidArgument;
  p.Rpad = padded_rows; p.qp = qdyt; p.ep = sdyt; p.qq = qht; p.eq = sht; p.o0 = dw2;
  launch<kDw2, true>(p, stream);
  return launch_status();
}
