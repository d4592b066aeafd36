// Persistent grouped GEMMs for the SwiGLU experts on MI355X (bf16 MFMA).
//
// Replaces the three torch._grouped_mm calls of
// torchtitan/models/common/moe.py:53-70 (_run_experts_grouped_mm) and their
// autograd. Expert e owns the rows [start_e, start_e + count_e) of the routed
// activations (start = exclusive cumsum of num_tokens_per_expert, moe.py:60).
//
// Every kernel computes, per expert, C[m][n] = sum_k P[m][k] * Q[n][k]:
//
//   mode        C (m x n)            P [m][k]         Q [n][k]              k
//   gate_up     [g|u] rows x 2H      x rows           w1/w3 rows            D
//   down        y rows x D           h rows           w2 rows               H
//   bwd_dgu     dh rows x H          dy rows          w2^T (H-contiguous)   D
//   bwd_dx      dx rows x D          dgu rows         [w1;w3]^T             2H
//   bwd_dw13    [dw1;dw3] 2H x D     dgu^T            x^T                   tokens
//   bwd_dw2     dw2 D x H            dy^T             h^T                   tokens
//
// Design (gfx950, 64-wide waves):
//  * Wave tiles of 64 x 128 (or 64 x 96) of v_mfma_f32_16x16x32_bf16 (fp32
//    accumulate), two waves per SIMD so each hides the other's LDS latency:
//    forward modes and dgu 4 waves / 128 x 256 block / two workgroups per CU,
//    dx and dW 8 waves / 128 x 512, 128 x 384 or 256 x 256 block / one
//    workgroup per CU (wider blocks copy fewer bytes per flop). k-step 32.
//  * Operands go HBM/L2 -> LDS with direct-to-LDS copies
//    (global_load_lds_dwordx4: each wave instruction fills 1 KB of LDS), so no
//    VGPRs stage the tiles and no ds_write is issued. Two or three LDS stages:
//    the copies of the next stages are in flight while stage k feeds the
//    MFMAs; one barrier per k-step. The copies are issued as inline asm and
//    waited for with explicit vmcnt, so the compiler neither serialises them
//    against the LDS reads nor adds waits of its own. Measured: the kernels
//    are bound by the latency of these copies (HBM and L2 round trips), not
//    by LDS or MFMA throughput.
//  * LDS layouts, both conflict-free for their fragment reads (measured on
//    gfx950, where a 16-byte read is served 8 lanes = 128 bytes at a time):
//      - K-contiguous operands: row-major 64-byte rows, 16-byte chunk kc of
//        row r at chunk kc ^ ((r >> 1) & 3); a copy instruction fills 16 rows,
//        four lanes per row (coalesced);
//      - M/N-contiguous operands (transposed weights, the dW operands):
//        k-major rows, 16-byte chunk c of k-row k at c ^ kswz(k); fragments
//        come from pairs of ds_read_b64_tr_b16 transposing reads.
//  * Persistent grid. Each workgroup derives the expert segments and
//    per-expert tile counts from num_tokens_per_expert in LDS (atomics-free
//    scan), so empty and heavily loaded experts need no host sync and no
//    padding. Workgroup ids are remapped so each XCD works on a contiguous
//    window of tiles (neighbouring tiles share an operand in its L2). In the
//    last m-tile of an expert, waves skip the MFMAs of 16-row blocks that hold
//    no routed rows.
//  * The K loop runs in ascending k in steps of 32 and each output element is
//    rounded to bf16 once, at the points the reference's bf16 autograd rounds;
//    the outputs are bit-identical to torch._grouped_mm and its autograd on
//    this GPU.
#include <cstring>
#include <type_traits>

#include "common.h"


namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmMaxE = 1024;

enum GemmMode : int {
  kFwdGateUp = 0,
  kFwdDown = 1,
  kBwdDgu = 2,
  kBwdDx = 3,
  kBwdDw13 = 4,
  kBwdDw2 = 5,
};

struct GemmParams {
  const int64_t* counts;  // [E]
  int64_t R;              // rows of the routed tensors; segments are clamped to it
  int E, D, H;
  const uint16_t* x;    // [R, D]
  const uint16_t* w1;   // [E, H, D]
  const uint16_t* w2;   // [E, D, H]
  const uint16_t* w3;   // [E, H, D]
  const uint16_t* h;    // [R, H]
  const uint16_t* g;    // [R, H]
  const uint16_t* u;    // [R, H]
  const uint16_t* dy;   // [R, D]
  const uint16_t* dgu;  // [R, 2H]: dg in [0, H), du in [H, 2H)
  uint16_t* out_g;
  uint16_t* out_u;
  uint16_t* out_h;
  uint16_t* out_y;
  uint16_t* out_dgu;
  uint16_t* out_dx;
  uint16_t* out_dw1;
  uint16_t* out_dw2;
  uint16_t* out_dw3;
  // w1 / w3 (and dw1 / dw3) row j of expert e at base + e * w13_estride + j * w13_rstride:
  // (H D, D) for separate [E, H, D] tensors; (2 H D, 2 D) with w3 = w1 + D for the
  // interleaved gate/linear rows of gpt-oss's mlp1_weight [E, 2H, D]
  int64_t w13_estride, w13_rstride;
  // gpt-oss expert epilogue (torchtitan/models/gpt_oss/moe.py:43-52, 92-122)
  const uint16_t* b1;  // mlp1_bias [E, 2H] bf16 (glu 2j, linear 2j + 1)
  const uint16_t* b2;  // mlp2_bias [E, D] bf16
  float limit;         // swiglu_limit as bf16
  float alpha;         // 1.702
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// Expert epilogue variants: the SwiGLU of moe.py:53-70 and gpt-oss's biased,
// clamped SwiGLU with interleaved mlp1 rows (gpt_oss/moe.py:43-52, 92-122).
enum ExpertAct : int { kSwiGLU = 0, kOssGLU = 1 };

// gpt-oss activation on bf16 values g (glu), u (linear), every op rounded to
// bf16 as the reference's bf16 tensor ops: clamp(g, max=L), clamp(u, -L, L),
// g * sigmoid(alpha g), times (u + 1). Returns the last product unrounded.
__device__ __forceinline__ float oss_glu(float g, float u, float L, float alpha) {
  const float xg = g > L ? L : g;                      // NaN passes, as torch.clamp
  const float xl = u < -L ? -L : (u > L ? L : u);
  const float s = round_bf(sigmoid_f(round_bf(xg * alpha)));
  return round_bf(xg * s) * round_bf(xl + 1.0f);
}
template <int MODE>
struct ModeTraits {
  static constexpr bool kRowGrouped = MODE <= kBwdDx;   // m = token rows of one expert
  static constexpr bool kPT = MODE >= kBwdDw13;          // P contiguous along m
  static constexpr bool kQT = MODE >= kBwdDgu;           // Q contiguous along n
};

// Interleave of the gate_up output columns: 16-column blocks alternate
// between g (w1) and u (w3), so a lane's SwiGLU operands sit in one wave.
__device__ __forceinline__ int gate_up_col(int nt, int n, int BN) {
  return nt * (BN / 2) + ((n >> 4) >> 1) * 16 + (n & 15);
}
__device__ __forceinline__ const uint16_t* gate_up_row(const GemmParams& p, int64_t e, int nt, int n, int BN) {
  return (((n >> 4) & 1) ? p.w3 : p.w1) + e * p.w13_estride + (int64_t)gate_up_col(nt, n, BN) * p.w13_rstride;
}

#define LDSP __attribute__((address_space(3)))
typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef short v8s_t __attribute__((ext_vector_type(8)));

// One wave-wide direct-to-LDS copy: lane i's 16 bytes at g land at LDS byte
// address lds + 16 i. Issued as inline asm so the compiler neither waits on it
// before unrelated LDS reads nor reorders it; the kernel waits with vmcnt.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" :: "v"(g), "{m0}"(lds) : "memory");
}
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* ptr) { return (uint32_t)(size_t)((LDSP T*)ptr); }

// Row-major LDS tile with rows of BK bf16 of k (64 or 128 bytes): element offset of
// 16-byte chunk kc of row r. 64-byte rows: chunk kc ^ ((r >> 1) & 3); 128-byte rows
// (whole cache lines per row): chunk kc ^ (r & 7).
template <int BK>
__device__ __forceinline__ int rm_off(int r, int kc) {
  if constexpr (BK == 32) return (r * 4 + (kc ^ ((r >> 1) & 3))) * 8;
  else return (r * 8 + (kc ^ (r & 7))) * 8;
}

// 16-byte chunk swizzle of a k-major tile row k (rows of 16 or more chunks):
// conflict-free for transposed fragment reads (32 lanes per LDS pass read 8 k-rows).
__device__ __forceinline__ int kswz(int k) { return 2 * ((k & 3) | ((k >> 1) & 4)); }
template <int ROWE>
__device__ __forceinline__ int km_off(int k, int n) { return k * ROWE + ((((n >> 3) ^ kswz(k)) << 3) | (n & 7)); }

// MFMA fragment (16 rows x 32 k, lane l: row l % 16, k 8 (l / 16) .. + 7) from a
// K-contiguous tile (row-major 64-byte rows).
template <int BK>
__device__ __forceinline__ bf16x8_t frag_rm(const uint16_t* tile, int row, int lane, int kh) {
  return *(const bf16x8_t*)(tile + rm_off<BK>(row, kh * 4 + (lane >> 4)));
}
// the same fragment from a k-major tile of ROWE elements per k-row, with two
// transposing reads (each lane supplies 4 consecutive rows of one k)
template <int ROWE>
__device__ __forceinline__ bf16x8_t frag_km(const uint16_t* tile, int row0, int lane) {
  const int g = lane >> 4, j = lane & 15;
  const int k = 8 * g + (j >> 2), n = row0 + 4 * (j & 3);
  const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDSP v4s_t*)(tile + km_off<ROWE>(k, n)));
  const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDSP v4s_t*)(tile + km_off<ROWE>(k + 4, n)));
  const v8s_t c = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, c);
}

__device__ const uint4 kZeroRow[64] = {};  // source of the zero rows past a segment

// TAIL: the n extent (and, for dW, the m extent) is not a multiple of the tile;
// compiled only for such shapes so that whole-tile shapes keep the tighter code.
template <int MODE, int NW, int WGM, int TM, int TN, int NS, bool SKIP, int OCC, int ACT, bool TAIL, int BKT>
__global__ __launch_bounds__(NW * 64, OCC) void grouped_gemm_kernel(GemmParams p) {
  using T = ModeTraits<MODE>;
  constexpr int WGN = NW / WGM;
  constexpr int WM = TM * 16, WN = TN * 16;
  constexpr int BM = WGM * WM, BN = WGN * WN, BK = BKT;
  static_assert(BK == 32 || (BK == 64 && !T::kPT && !T::kQT), "k-steps of 64 for k-contiguous operands only");
  constexpr int RPC = 512 / BK;  // tile rows per 1 KB copy (k-contiguous tiles)
  constexpr int KH = BK / 32;    // MFMA k-steps per stage
  constexpr int CPW_P = BM * BK / 512 / NW, CPW_Q = BN * BK / 512 / NW;  // 1 KB copies per wave and stage
  static_assert(CPW_P * 512 * NW == BM * BK && CPW_Q * 512 * NW == BN * BK, "copies per wave");
  constexpr int CPW = CPW_P + CPW_Q;
  constexpr int kIlvSpan = 4;  // pipelined k-steps: the slots the next stage's copies spread over
  constexpr int CHP = BM / 8, CHQ = BN / 8;          // 16-byte chunks per k-row (k-major tiles)
  static_assert(BM % 64 == 0 && BN % 64 == 0 && CPW <= 30, "tile");
  static_assert(TN % 2 == 0 && (MODE != kFwdGateUp || TN % 4 == 0), "epilogue block pairs");
  // kswz flips chunk bits 1-3: a k-major row must hold whole groups of 16 chunks
  static_assert((!T::kPT || BM % 128 == 0) && (!T::kQT || BN % 128 == 0), "k-major tile rows");
  __shared__ __attribute__((aligned(1024))) uint16_t sP[NS][BM * BK];
  __shared__ __attribute__((aligned(1024))) uint16_t sQ[NS][BN * BK];
  __shared__ int s_seg[kGemmMaxE + 1];
  __shared__ int s_tile[kGemmMaxE + 1];
  __shared__ int s_tmp[8];

  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv / WGN, wn = wv % WGN;
  const int E = p.E, D = p.D, H = p.H;
  int Ntot = 0, Kfix = 0, Mfix = 0;
  if (MODE == kFwdGateUp) { Ntot = 2 * H; Kfix = D; }
  if (MODE == kFwdDown) { Ntot = D; Kfix = H; }
  if (MODE == kBwdDgu) { Ntot = H; Kfix = D; }
  if (MODE == kBwdDx) { Ntot = D; Kfix = 2 * H; }
  if (MODE == kBwdDw13) { Ntot = D; Mfix = 2 * H; }
  if (MODE == kBwdDw2) { Ntot = H; Mfix = D; }
  // D and H are multiples of 64: the last n-tile (and, for dW, m-tile) may be
  // partial; its copies past the edge read the zero row and its stores are skipped
  const int NT = (Ntot + BN - 1) / BN;
  const int MT = T::kRowGrouped ? 0 : (Mfix + BM - 1) / BM;

  {
    int cnt[4], tl[4], seg[4], tst[4];
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
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      tl[i] = (e < E) ? (T::kRowGrouped ? ((cnt[i] + BM - 1) / BM) * NT : MT * NT) : 0;
    }
    const int rtot = block_exclusive_scan4(cnt, seg, s_tmp);
    const int ttot = block_exclusive_scan4(tl, tst, s_tmp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      if (e < E) { s_seg[e] = seg[i]; s_tile[e] = tst[i]; }
    }
    if (tid == 0) { s_seg[E] = rtot; s_tile[E] = ttot; }
    __syncthreads();
  }
  const int total_tiles = s_tile[E];
  const int G = gridDim.x;
  const int lb = (G % 8 == 0) ? ((int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3)) : (int)blockIdx.x;
  const int ml = lane & 15, nq = (lane >> 4) * 4;
  // copy-lane maps. K-contiguous tile: one copy = 16 rows x 64 B, lane i -> row i >> 2,
  // chunk (i & 3) ^ ((row >> 1) & 3). k-major tile: one copy = 1 KB of k-rows, lane i ->
  // k-row i / (ROWB / 16), chunk (i % (ROWB / 16)) ^ kswz(k).
  const int dr = BK == 32 ? lane >> 2 : lane >> 3;
  const int dc = BK == 32 ? (lane & 3) ^ ((dr >> 1) & 3) : (lane & 7) ^ (dr & 7);

  // ---- tiles ----
  struct TileRef { int e, seg0, seg1, mt, nt, nk; };
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
    if (T::kRowGrouped) {
      const int mtiles = (r.seg1 - r.seg0 + BM - 1) / BM;
      r.nt = local / mtiles;
      r.mt = local - r.nt * mtiles;
    } else if (MODE == kBwdDw13 && MT >= 16 && MT % 4 == 0) {
      // blocks of 4 m-tiles by every n-tile, so that the 32 consecutive tiles one XCD
      // runs together share 4 dgu slices and 8 x slices instead of 16 and 2 (DSv3,
      // 16 m-tiles by 28 n-tiles per expert: 6.85 -> 6.37 ms; no gain for dw2, and
      // at 8 m-tiles, Kimi, the plain order already shares both operands)
      const int blk = local / (NT * 4), rem = local - blk * NT * 4;
      r.nt = rem / 4;
      r.mt = blk * 4 + (rem - r.nt * 4);
    } else {
      r.nt = local / MT;
      r.mt = local - r.nt * MT;
    }
    const int Ktot = T::kRowGrouped ? Kfix : (r.seg1 - r.seg0);
    r.nk = (Ktot + BK - 1) / BK;
    return r;
  };

  // ---- per-lane copy sources of the tile being copied (copy c of this wave covers
  // LDS bytes [1 KB (wv CPW_X + c), +1 KB)) ----
  const uint16_t* srcP[CPW_P];
  const uint16_t* srcQ[CPW_Q];
  const uint16_t* srcQ3[CPW_Q];  // dx: the w3 half of the k range
  int klP[CPW_P], klQ[CPW_Q];    // k-major copies: the k-row this lane fills (P rows: the token row)
  bool inP[CPW_P], inQ[CPW_Q];   // the copied m / n lies inside the matrix
  int64_t stepP = BK, stepQ = BK;  // element advance per k-step
  if constexpr (T::kPT) stepP = (int64_t)BK * ((MODE == kBwdDw13) ? 2 * H : D);
  if constexpr (MODE == kBwdDgu) stepQ = (int64_t)BK * H;
  if constexpr (MODE == kBwdDx) stepQ = (int64_t)BK * p.w13_rstride;
  if constexpr (MODE == kBwdDw13) stepQ = (int64_t)BK * D;
  if constexpr (MODE == kBwdDw2) stepQ = (int64_t)BK * H;
  auto setup = [&](const TileRef& r) {
    const int64_t e64 = r.e;
    const int row0 = r.seg0 + r.mt * BM;
    if constexpr (!T::kPT) {
      const uint16_t* pb;
      int ldp;
      if (MODE == kFwdGateUp) { pb = p.x; ldp = D; }
      else if (MODE == kFwdDown) { pb = p.h; ldp = H; }
      else if (MODE == kBwdDgu) { pb = p.dy; ldp = D; }
      else { pb = p.dgu; ldp = 2 * H; }
#pragma unroll
      for (int b = 0; b < CPW_P; ++b) {
        const int rr = row0 + (wv * CPW_P + b) * RPC + dr;
        srcP[b] = pb + (int64_t)rr * ldp + dc * 8;
        klP[b] = rr;  // rows past the segment copy the zero row
        inP[b] = true;
      }
    } else {
      const uint16_t* pb = (MODE == kBwdDw13) ? p.dgu : p.dy;
      const int ldp = (MODE == kBwdDw13) ? 2 * H : D;
#pragma unroll
      for (int b = 0; b < CPW_P; ++b) {
        const int slot = (wv * CPW_P + b) * 64 + lane;
        const int kl = slot / CHP;
        const int c = (slot % CHP) ^ kswz(kl);
        srcP[b] = pb + (int64_t)(r.seg0 + kl) * ldp + r.mt * BM + c * 8;
        klP[b] = kl;
        inP[b] = r.mt * BM + c * 8 < Mfix;
      }
    }
    if constexpr (!T::kQT) {
#pragma unroll
      for (int b = 0; b < CPW_Q; ++b) {
        const int n = (wv * CPW_Q + b) * RPC + dr;
        inQ[b] = (MODE == kFwdGateUp) ? gate_up_col(r.nt, n, BN) < H : r.nt * BN + n < D;
        const uint16_t* rowp = (MODE == kFwdGateUp) ? gate_up_row(p, e64, r.nt, n, BN)
                                                     : p.w2 + (e64 * D + r.nt * BN + n) * (int64_t)H;
        srcQ[b] = rowp + dc * 8;
        klQ[b] = 0;
      }
    } else {
      const uint16_t* qb;
      int64_t ldq;
      if (MODE == kBwdDgu) { qb = p.w2 + e64 * D * (int64_t)H; ldq = H; }        // rows k of w2[e] (D x H)
      else if (MODE == kBwdDx) { qb = p.w1 + e64 * p.w13_estride; ldq = p.w13_rstride; }  // rows k of w1[e], then w3[e]
      else if (MODE == kBwdDw13) { qb = p.x + (int64_t)r.seg0 * D; ldq = D; }
      else { qb = p.h + (int64_t)r.seg0 * H; ldq = H; }
#pragma unroll
      for (int b = 0; b < CPW_Q; ++b) {
        const int slot = (wv * CPW_Q + b) * 64 + lane;
        const int kl = slot / CHQ;
        const int c = (slot % CHQ) ^ kswz(kl);
        const int64_t off = (int64_t)kl * ldq + r.nt * BN + c * 8;
        srcQ[b] = qb + off;
        if (MODE == kBwdDx) srcQ3[b] = p.w3 + e64 * p.w13_estride + off;
        klQ[b] = kl;
        inQ[b] = r.nt * BN + c * 8 < Ntot;
      }
    }
  };

  // copy c (P copies first, then Q) of stage kt of tile r into LDS buffer s
  auto issue_copy = [&](const TileRef& r, int kt, int s, int c) {
    const int k0 = kt * BK;
    if (c < CPW_P) {
      const int b = c;
      const uint16_t* src = srcP[b] + kt * stepP;
      if constexpr (T::kPT) {
        if (r.seg0 + k0 + klP[b] >= r.seg1 || (TAIL && !inP[b])) src = (const uint16_t*)kZeroRow;
      } else {
        if (klP[b] >= r.seg1) src = (const uint16_t*)kZeroRow;
      }
      dma16(src, lds_addr(&sP[s][(wv * CPW_P + b) * 512]));
    } else {
      const int b = c - CPW_P;
      const uint16_t* src = srcQ[b] + kt * stepQ;
      if constexpr (MODE == kBwdDx) {
        if (k0 >= H) src = srcQ3[b] + (int64_t)(k0 - H) * p.w13_rstride;
      }
      if constexpr (MODE >= kBwdDw13) {
        if (r.seg0 + k0 + klQ[b] >= r.seg1) src = (const uint16_t*)kZeroRow;
      }
      if (TAIL && !inQ[b]) src = (const uint16_t*)kZeroRow;
      dma16(src, lds_addr(&sQ[s][(wv * CPW_Q + b) * 512]));
    }
  };
  // stage kt of tile r into LDS buffer s
  auto issue = [&](const TileRef& r, int kt, int s) {
#pragma unroll
    for (int c = 0; c < CPW; ++c) issue_copy(r, kt, s, c);
  };

  // One stream of copy stages across this workgroup's tiles: the copy cursor
  // (tile ct_i, step ik) runs NS - 1 stages ahead of the MFMAs, through tile
  // boundaries, so the next tile's first stages are in flight while this tile's
  // epilogue runs. Stage g uses LDS buffer g % NS. Tiles without k-steps (dW of
  // an expert without tokens) have no stages.
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
  auto advance = [&]() {
    ++gi;
    if (++ik == ir.nk) seek(ct_i + G);
  };
  auto issue_next = [&]() {
    issue(ir, ik, gi % NS);
    advance();
  };
  seek(lb);
#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (ct_i < total_tiles) issue_next();

  for (int t = lb; t < total_tiles; t += G) {
    const TileRef cr = decode(t);
    const int e = cr.e;
    const int64_t e64 = e;
    const int seg1 = cr.seg1, mt = cr.mt, nt = cr.nt, nk = cr.nk;
    const int row0 = cr.seg0 + mt * BM;

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int tmv = T::kRowGrouped ? min(TM, max(0, (seg1 - (row0 + wm * WM) + 15) >> 4)) : TM;
    const int kt_half = (MODE == kBwdDx) ? H / BK : -1;

    // dx = bf16(dg . w1) + bf16(du . w3), the sum of the two bf16 gradients autograd
    // accumulates into x: after the w1 half of the k range the accumulators are
    // rounded to bf16 and parked, then restarted for w3. Wave tiles up to 64 x 96
    // park in registers (2 TM TN VGPRs); wider ones, which have no registers to
    // spare, park in the dx rows themselves and read them back in the epilogue.
    constexpr bool kParkRegs = TM * TN <= 24;
    uint32_t park[kParkRegs ? TM : 1][kParkRegs ? TN : 1][2];
    auto park_dx_half = [&]() {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if constexpr (kParkRegs) {
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            park[i][j][0] = pack_bf2(acc[i][j][0], acc[i][j][1]);
            park[i][j][1] = pack_bf2(acc[i][j][2], acc[i][j][3]);
          }
        } else {
          // 64-byte row pieces of the dx rows (read back the same way in the epilogue)
#pragma unroll
          for (int jp = 0; jp < TN / 2; ++jp) {
            const float lo[4] = {acc[i][2 * jp][0], acc[i][2 * jp][1], acc[i][2 * jp][2], acc[i][2 * jp][3]};
            const float hi[4] = {acc[i][2 * jp + 1][0], acc[i][2 * jp + 1][1], acc[i][2 * jp + 1][2],
                                 acc[i][2 * jp + 1][3]};
            const uint4 sv = span64(pack4(lo), pack4(hi), lane);
            const int n = nt * BN + wn * WN + jp * 32 + 8 * (lane >> 4);
            if (r < seg1 && (!TAIL || n < D)) *(uint4*)(p.out_dx + (int64_t)r * D + n) = sv;
          }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    };

    auto run = [&](auto full) {
      auto compute = [&](int s) {
        const uint16_t* cP = sP[s];
        const uint16_t* cQ = sQ[s];
#pragma unroll
        for (int kh = 0; kh < KH; ++kh) {
          bf16x8_t af[TM];
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            if (!decltype(full)::value && i >= tmv) continue;
            if constexpr (T::kPT) af[i] = frag_km<BM>(cP, wm * WM + i * 16, lane);
            else af[i] = frag_rm<BK>(cP, wm * WM + i * 16 + ml, lane, kh);
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            bf16x8_t bq;
            if constexpr (T::kQT) bq = frag_km<BN>(cQ, wn * WN + j * 16, lane);
            else bq = frag_rm<BK>(cQ, wn * WN + j * 16 + ml, lane, kh);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
              if (!decltype(full)::value && i >= tmv) continue;
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq, af[i], acc[i][j], 0, 0, 0);
            }
          }
        }
      };
      // Software-pipelined k-step: slots of 2 x TM MFMAs (two 16-column blocks of one
      // 32-wide k half); each slot first reads the next slot's B fragments from LDS,
      // then issues its MFMAs, then its share of the next stage's copies (nx: there is
      // a next stage, into LDS buffer sn), which are spread over the first kIlvSpan
      // slots. In the plain schedule every wave issues all its copies right after the
      // barrier and each pair of B fragments is waited for right before its MFMAs: a
      // copy issue that stalls on a full texture queue then holds every MFMA of the
      // wave behind it, and the LDS latency is exposed once per slot. Same MFMAs in
      // the same order as the plain schedule, so the accumulators are bit-identical.
      auto compute_ilv = [&](int s, bool nx, int sn) {
        const uint16_t* cP = sP[s];
        const uint16_t* cQ = sQ[s];
        constexpr int JP = TN / 2, NSL = KH * JP, SPAN = kIlvSpan < NSL ? kIlvSpan : NSL;
        bf16x8_t af[TM], bq[2][2];
        auto load_a = [&](int kh) {
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            if (!decltype(full)::value && i >= tmv) continue;
            if constexpr (T::kPT) af[i] = frag_km<BM>(cP, wm * WM + i * 16, lane);
            else af[i] = frag_rm<BK>(cP, wm * WM + i * 16 + ml, lane, kh);
          }
        };
        auto load_b = [&](int sl) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int j = 2 * (sl % JP) + h;
            if constexpr (T::kQT) bq[sl & 1][h] = frag_km<BN>(cQ, wn * WN + j * 16, lane);
            else bq[sl & 1][h] = frag_rm<BK>(cQ, wn * WN + j * 16 + ml, lane, sl / JP);
          }
        };
        load_a(0);
        load_b(0);
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl) {
          const int kh = sl / JP, jp = sl % JP;
          if (sl > 0 && jp == 0) load_a(kh);
          if (sl + 1 < NSL) load_b(sl + 1);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
              if (!decltype(full)::value && i >= tmv) continue;
              acc[i][2 * jp + h] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[sl & 1][h], af[i], acc[i][2 * jp + h], 0, 0, 0);
            }
          }
#pragma unroll
          for (int c = 0; c < CPW; ++c)
            if (nx && c * SPAN / CPW == sl) issue_copy(ir, ik, sn, c);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      // Pipelined: the tiles with 64-wide k-steps (forward modes only). With 32-wide
      // k-steps (the 128 x 256 forward tile, dgu, dx, dW) the plain schedule measured
      // faster. Waves with a partial row block keep the plain schedule too (their
      // conditional MFMAs with the pipeline's registers spill).
      constexpr bool kIlv = BK == 64 && decltype(full)::value;
      for (int kt = 0; kt < nk; ++kt) {
        // stage gc has landed in every wave once at most the one stage issued after it
        // is outstanding (stores of the previous epilogue only add to the count); the
        // barrier also retires every wave's reads of the buffer refilled next
        if (NS == 3 && gi - gc >= 2) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" :: "n"(CPW) : "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if constexpr (kIlv) {
          const bool nx = ct_i < total_tiles;
          if (MODE == kBwdDx && ACT == kSwiGLU && kt == kt_half) park_dx_half();
          compute_ilv(gc % NS, nx, gi % NS);
          if (nx) advance();
        } else {
          if (ct_i < total_tiles) issue_next();
          if (MODE == kBwdDx && ACT == kSwiGLU && kt == kt_half) park_dx_half();
          if (decltype(full)::value || tmv > 0) compute(gc % NS);
        }
        ++gc;
      }
    };
    if (!SKIP || tmv == TM) run(std::true_type{});
    else run(std::false_type{});

    // ---- epilogue: lane holds C[m = .. + ml][n = .. + nq + 0..3] ----
    // Each lane produces 4 columns per 16-column block; pairs of blocks are stored
    // as 64-byte row pieces (span64), at column 32 jp + 8 (lane / 16) of the wave's span.
    const int g8 = 8 * (lane >> 4);
    // gpt-oss biases: one per column, so loaded once per tile before the first store
    // (a load issued after a store, which may alias it, waits behind it)
    uint4 bias1[ACT == kOssGLU && MODE == kFwdGateUp ? TN / 2 : 1];
    uint2 bias2[ACT == kOssGLU && MODE == kFwdDown ? TN : 1];
    if constexpr (ACT == kOssGLU && MODE == kFwdGateUp) {
#pragma unroll
      for (int jj = 0; jj < TN / 2; ++jj) {
        const int hc = nt * (BN / 2) + wn * (WN / 2) + jj * 16 + nq;
        bias1[jj] = (!TAIL || hc < H) ? *(const uint4*)(p.b1 + e64 * 2 * H + 2 * hc) : make_uint4(0, 0, 0, 0);
      }
    }
    if constexpr (ACT == kOssGLU && MODE == kFwdDown) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = nt * BN + wn * WN + j * 16 + nq;
        bias2[j] = (!TAIL || n < D) ? *(const uint2*)(p.b2 + e64 * D + n) : make_uint2(0, 0);
      }
    }
    if (MODE == kFwdGateUp) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        // one 16-row block's columns, silu in its fast or its dividing form
        auto block = [&](auto fast_c) {
          constexpr bool kFast = decltype(fast_c)::value;
#pragma unroll
          for (int jp = 0; jp < TN / 4; ++jp) {
            uint2 pg[2], pu[2], ph[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int jj = 2 * jp + h2;
              // Column pairs are rounded to packed bf16 once; the fp32 operands of the
              // activation are read back from the packed words (exact), so each value
              // takes one NaN-canonicalizing conversion. The epilogue is VALU-bound:
              // rounding each value to fp32-held bf16 and then packing it again cost
              // a third of its instructions.
              uint32_t gq[2], uq[2], hq[2];
#pragma unroll
              for (int q2 = 0; q2 < 2; ++q2) {
                const int q = 2 * q2;
                uint32_t gw = pack_bf2(acc[i][2 * jj][q], acc[i][2 * jj][q + 1]);
                uint32_t uw = pack_bf2(acc[i][2 * jj + 1][q], acc[i][2 * jj + 1][q + 1]);
                if constexpr (ACT == kOssGLU) {
                  // h1 = bf16(x . mlp1^T) + bias (bf16 add), then the clamped SwiGLU;
                  // bias word of column c: (glu, linear)
                  const uint4 bw = bias1[jj];
                  const uint32_t bb[4] = {bw.x, bw.y, bw.z, bw.w};
                  gw = pack_bf2(bf_lo(gw) + bf_lo(bb[q]), bf_hi(gw) + bf_lo(bb[q + 1]));
                  uw = pack_bf2(bf_lo(uw) + bf_hi(bb[q]), bf_hi(uw) + bf_hi(bb[q + 1]));
                  hq[q2] = pack_bf2(oss_glu(bf_lo(gw), bf_lo(uw), p.limit, p.alpha),
                                    oss_glu(bf_hi(gw), bf_hi(uw), p.limit, p.alpha));
                } else {
                  const float g0 = bf_lo(gw), g1 = bf_hi(gw);
                  const uint32_t sw = pack_bf2(silu_sig<kFast>(g0, silu_den(g0)).silu,
                                               silu_sig<kFast>(g1, silu_den(g1)).silu);  // bf16(silu(g))
                  hq[q2] = pack_bf2(bf_lo(sw) * bf_lo(uw), bf_hi(sw) * bf_hi(uw));
                }
                gq[q2] = gw;
                uq[q2] = uw;
              }
              pg[h2] = make_uint2(gq[0], gq[1]);
              pu[h2] = make_uint2(uq[0], uq[1]);
              ph[h2] = make_uint2(hq[0], hq[1]);
            }
            const int hc = nt * (BN / 2) + wn * (WN / 2) + jp * 32 + g8;
            const uint4 sg = span64(pg[0], pg[1], lane), su = span64(pu[0], pu[1], lane),
                        sh = span64(ph[0], ph[1], lane);
            if (TAIL && hc >= H) continue;
            const int64_t off = (int64_t)r * H + hc;
            *(uint4*)(p.out_g + off) = sg;
            *(uint4*)(p.out_u + off) = su;
            *(uint4*)(p.out_h + off) = sh;
          }
        };
        if (r < seg1) {
          if constexpr (ACT == kSwiGLU) {
            // the range of the block's gate values, taken before their rounding to
            // bf16, which keeps them inside it
            float g_min = acc[i][0][0], g_max = acc[i][0][0];
#pragma unroll
            for (int jj = 0; jj < TN / 2; ++jj)
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                g_min = fminf(g_min, acc[i][2 * jj][q]);
                g_max = fmaxf(g_max, acc[i][2 * jj][q]);
              }
            if (silu_fast_wave(g_min, g_max)) block(std::true_type{});
            else block(std::false_type{});
          } else {
            block(std::true_type{});
          }
        }
      }
    } else if (MODE == kFwdDown || MODE == kBwdDx) {
      uint16_t* outp = (MODE == kFwdDown) ? p.out_y : p.out_dx;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
#pragma unroll
          for (int jp = 0; jp < TN / 2; ++jp) {
            if constexpr (MODE == kBwdDx && ACT == kSwiGLU && !kParkRegs) {
              // the w3 half, rounded to bf16, in the span layout; the parked w1 half is
              // read back from the dx rows as 16-byte pieces
              const float lo[4] = {acc[i][2 * jp][0], acc[i][2 * jp][1], acc[i][2 * jp][2], acc[i][2 * jp][3]};
              const float hi[4] = {acc[i][2 * jp + 1][0], acc[i][2 * jp + 1][1], acc[i][2 * jp + 1][2],
                                   acc[i][2 * jp + 1][3]};
              const uint4 sv = span64(pack4(lo), pack4(hi), lane);
              const int n = nt * BN + wn * WN + jp * 32 + g8;
              if (TAIL && n >= D) continue;
              uint16_t* dst = outp + (int64_t)r * D + n;
              const uint4 pw = *(const uint4*)dst;
              const uint32_t a4[4] = {sv.x, sv.y, sv.z, sv.w}, b4[4] = {pw.x, pw.y, pw.z, pw.w};
              uint32_t o4[4];
#pragma unroll
              for (int q = 0; q < 4; ++q)
                o4[q] = pack_bf2(bf_lo(b4[q]) + bf_lo(a4[q]), bf_hi(b4[q]) + bf_hi(a4[q]));
              *(uint4*)dst = make_uint4(o4[0], o4[1], o4[2], o4[3]);
              continue;
            }
            uint2 pv[2];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int j = 2 * jp + h2;
              const int n = nt * BN + wn * WN + j * 16 + nq;
              const bool in = !TAIL || n < D;
              float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
              if (MODE == kFwdDown && ACT == kOssGLU) {  // bf16(h . mlp2^T) + mlp2_bias (bf16 add)
                const uint2 bw = bias2[j];
                v[0] = round_bf(v[0]) + bf_lo(bw.x);
                v[1] = round_bf(v[1]) + bf_hi(bw.x);
                v[2] = round_bf(v[2]) + bf_lo(bw.y);
                v[3] = round_bf(v[3]) + bf_hi(bw.y);
              }
              if constexpr (MODE == kBwdDx && ACT == kSwiGLU && kParkRegs) {
                const uint2 pw = make_uint2(park[i][j][0], park[i][j][1]);
                v[0] = bf_lo(pw.x) + round_bf(v[0]);
                v[1] = bf_hi(pw.x) + round_bf(v[1]);
                v[2] = bf_lo(pw.y) + round_bf(v[2]);
                v[3] = bf_hi(pw.y) + round_bf(v[3]);
              }
              pv[h2] = pack4(v);
            }
            const int n = nt * BN + wn * WN + jp * 32 + g8;
            const uint4 sv = span64(pv[0], pv[1], lane);
            if (TAIL && n >= D) continue;
            *(uint4*)(outp + (int64_t)r * D + n) = sv;
          }
        }
      }
    } else if (MODE == kBwdDgu) {
      // dh = bf16(dy . w2) is gathered into the 64-byte span layout first, so g and u
      // are read, and dg and du written, as 16-byte pieces of 64 contiguous bytes per row.
      // The g and u pieces of a 16-row block are loaded together, in one batch before
      // the block's stores: one exposed memory round trip per 16-row block instead of
      // one per piece (a load issued after a store, which may alias it, waits behind it).
      uint4 gbuf[1][TN / 2], ubuf[1][TN / 2];
      auto load_gu = [&](int i, int b) {
        const int r = row0 + wm * WM + i * 16 + ml;
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          const int hh = nt * BN + wn * WN + jp * 32 + g8;
          if (r < seg1 && (!TAIL || hh < H)) {
            const int64_t off = (int64_t)r * H + hh;
            gbuf[b][jp] = *(const uint4*)(p.g + off);
            ubuf[b][jp] = *(const uint4*)(p.u + off);
          }
        }
      };
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        load_gu(i, 0);
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
#pragma unroll
          for (int jp = 0; jp < TN / 2; ++jp) {
            const float lo[4] = {acc[i][2 * jp][0], acc[i][2 * jp][1], acc[i][2 * jp][2], acc[i][2 * jp][3]};
            const float hi[4] = {acc[i][2 * jp + 1][0], acc[i][2 * jp + 1][1], acc[i][2 * jp + 1][2],
                                 acc[i][2 * jp + 1][3]};
            const uint4 sdh = span64(pack4(lo), pack4(hi), lane);
            const int hh = nt * BN + wn * WN + jp * 32 + g8;
            if (TAIL && hh >= H) continue;
            const uint4 gw = gbuf[0][jp];
            const uint4 uw = ubuf[0][jp];
            const uint32_t dhw[4] = {sdh.x, sdh.y, sdh.z, sdh.w};
            const uint32_t gww[4] = {gw.x, gw.y, gw.z, gw.w};
            const uint32_t uww[4] = {uw.x, uw.y, uw.z, uw.w};
            float dg[8], du[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              const float dh = (q & 1) ? bf_hi(dhw[q >> 1]) : bf_lo(dhw[q >> 1]);
              const float gv = (q & 1) ? bf_hi(gww[q >> 1]) : bf_lo(gww[q >> 1]);
              const float uv = (q & 1) ? bf_hi(uww[q >> 1]) : bf_lo(uww[q >> 1]);
              if constexpr (ACT == kSwiGLU) {
                // column pairs: the two bf16 roundings of a pair are one conversion
                // (the epilogue is VALU-bound), read back exactly from the packed word
                if (q & 1) continue;
                const float dh1 = bf_hi(dhw[q >> 1]), gv1 = bf_hi(gww[q >> 1]), uv1 = bf_hi(uww[q >> 1]);
                const float d0 = silu_den(gv), d1 = silu_den(gv1);
                SiluSig f0, f1;
                if (silu_fast_wave(fminf(gv, gv1), fmaxf(gv, gv1))) {
                  f0 = silu_sig<true>(gv, d0);
                  f1 = silu_sig<true>(gv1, d1);
                } else {
                  f0 = silu_sig<false>(gv, d0);
                  f1 = silu_sig<false>(gv1, d1);
                }
                const uint32_t slw = pack_bf2(f0.silu, f1.silu);   // bf16(silu(g))
                const uint32_t dsw = pack_bf2(dh * uv, dh1 * uv1);  // bf16(dh . u)
                du[q] = dh * bf_lo(slw);
                du[q + 1] = dh1 * bf_hi(slw);
                const float sg = f0.sig, sg1 = f1.sig;
                dg[q] = bf_lo(dsw) * sg * (1.0f + gv * (1.0f - sg));
                dg[q + 1] = bf_hi(dsw) * sg1 * (1.0f + gv1 * (1.0f - sg1));
              } else {
                // autograd of oss_glu, each bf16 op's gradient rounded to bf16
                const float L = p.limit, al = p.alpha;
                const float xg = gv > L ? L : gv;
                const float xl = uv < -L ? -L : (uv > L ? L : uv);
                const float s = round_bf(sigmoid_f(round_bf(xg * al)));
                const float og = round_bf(xg * s);
                const float da = round_bf(dh * round_bf(xl + 1.0f));  // d(glu output)
                const float dl = round_bf(dh * og);                    // d(linear + 1)
                const float ds = round_bf(da * xg);                    // d(sigmoid output)
                const float dz = round_bf((ds * (1.0f - s)) * s);      // sigmoid_backward
                const float dxg = round_bf(da * s) + round_bf(dz * al);
                dg[q] = gv <= L ? dxg : 0.f;                           // clamp(max=L) backward
                du[q] = (uv >= -L && uv <= L) ? dl : 0.f;              // clamp(-L, L) backward
              }
            }
            const int64_t o2 = (int64_t)r * (2 * H) + hh;
            *(uint4*)(p.out_dgu + o2) = make_uint4(pack_bf2(dg[0], dg[1]), pack_bf2(dg[2], dg[3]),
                                                   pack_bf2(dg[4], dg[5]), pack_bf2(dg[6], dg[7]));
            *(uint4*)(p.out_dgu + o2 + H) = make_uint4(pack_bf2(du[0], du[1]), pack_bf2(du[2], du[3]),
                                                       pack_bf2(du[4], du[5]), pack_bf2(du[6], du[7]));
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = mt * BM + wm * WM + i * 16 + ml;
        if (TAIL && m >= Mfix) continue;
        uint16_t* rowp;
        if (MODE == kBwdDw13)
          rowp = (m < H) ? p.out_dw1 + e64 * p.w13_estride + m * p.w13_rstride
                         : p.out_dw3 + e64 * p.w13_estride + (m - H) * p.w13_rstride;
        else
          rowp = p.out_dw2 + (e64 * D + m) * (int64_t)H;
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          const float lo[4] = {acc[i][2 * jp][0], acc[i][2 * jp][1], acc[i][2 * jp][2], acc[i][2 * jp][3]};
          const float hi[4] = {acc[i][2 * jp + 1][0], acc[i][2 * jp + 1][1], acc[i][2 * jp + 1][2],
                               acc[i][2 * jp + 1][3]};
          const uint4 sv = span64(pack4(lo), pack4(hi), lane);
          const int n = nt * BN + wn * WN + jp * 32 + g8;
          if (TAIL && n >= Ntot) continue;
          *(uint4*)(rowp + n) = sv;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int g_cu_count[64];

static int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cu_count[dev] = n;
  }
  return g_cu_count[dev];
}

static int persistent_grid(int64_t max_tiles, int per_cu) {
  int64_t g = (int64_t)cu_count() * per_cu;
  if (g > max_tiles) g = max_tiles;
  if (g >= 8) g -= g % 8;
  return (int)(g < 1 ? 1 : g);
}

// One launch of grouped_gemm_kernel with NW waves in WGM x (NW / WGM), wave
// tiles (16 TM) x (16 TN), NS LDS stages and OCC workgroups per CU.
template <int MODE, int NW, int WGM, int TM, int TN, int NS, bool SKIP, int OCC, int ACT, int BKT = 32>
static void launch_cfg(const GemmParams& p, int64_t R, hipStream_t stream) {
  constexpr int BM = WGM * TM * 16, BN = (NW / WGM) * TN * 16;
  auto cdiv = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
  int64_t max_tiles;
  if (MODE == kFwdGateUp) max_tiles = (R / BM + p.E) * cdiv(2 * p.H, BN);
  else if (MODE == kFwdDown || MODE == kBwdDx) max_tiles = (R / BM + p.E) * cdiv(p.D, BN);
  else if (MODE == kBwdDgu) max_tiles = (R / BM + p.E) * cdiv(p.H, BN);
  else if (MODE == kBwdDw13) max_tiles = (int64_t)p.E * cdiv(2 * p.H, BM) * cdiv(p.D, BN);
  else max_tiles = (int64_t)p.E * cdiv(p.D, BM) * cdiv(p.H, BN);
  bool tail;
  if (MODE == kFwdGateUp) tail = (2 * p.H) % BN != 0;
  else if (MODE == kFwdDown || MODE == kBwdDx) tail = p.D % BN != 0;
  else if (MODE == kBwdDgu) tail = p.H % BN != 0;
  else if (MODE == kBwdDw13) tail = (2 * p.H) % BM != 0 || p.D % BN != 0;
  else tail = p.D % BM != 0 || p.H % BN != 0;
  const dim3 grid(persistent_grid(max_tiles, OCC)), block(NW * 64);
  if (tail)
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE, NW, WGM, TM, TN, NS, SKIP, OCC, ACT, true, BKT>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<MODE, NW, WGM, TM, TN, NS, SKIP, OCC, ACT, false, BKT>), grid, block, 0, stream, p);
}

// Tile per mode (measured at the Kimi and DSv3 shapes). The forward modes run
// 128 x 256 tiles, four waves, two workgroups per CU; gate_up over a long
// contraction (D >= 4096) runs the same tile as eight 64 x 64 waves with 64-wide
// k-steps (whole 128-byte rows per copy) and three stages at one workgroup per CU
// (DSv3, D = 7168: 6.25 -> 5.46 ms; at D = 2304 it is 6 % slower). 256 x 256 tiles of
// eight 64 x 128 waves with 64-wide k-steps, two stages, one workgroup per CU pay where
// the experts are tall, from 512 rows per expert on average, with either epilogue: down
// (Kimi, 512 rows: 0.81 -> 0.76-0.77 ms in the layer step; gpt-oss-20b, 2048 rows, H = 2880:
// 1.21-1.23 -> 1.04-1.16 ms; at DSv3, 256 rows, 6 % slower) and gate_up (Kimi 1.58-1.59 ->
// 1.54-1.55 ms in the layer step; 32K Kimi tokens, 1024 rows: 2.95 -> 2.72 ms; gpt-oss-20b
// 2.55 -> 2.27-2.44 ms). Both 64-wide configurations run the software-pipelined
// k-step (compute_ilv); down over a long contraction with short experts (H >= 2048,
// DSv3) takes gate_up's long-contraction tile. dgu runs the
// forward tile too: its epilogue reads g and u and writes dg and du, and with two
// workgroups per CU one's epilogue overlaps the other's MFMAs (against one
// eight-wave 128 x 512 workgroup: DSv3 3.15 -> 2.81 ms, Kimi -1.5 %). dx and dW run
// one eight-wave workgroup per CU with three LDS stages and wider tiles, which
// halves the copy traffic per flop of the dW operands: 128 x 384 (dx, D a multiple
// of 384), 128 x 512 (dx, D a multiple of 512), 256 x 256 (dW). D and H are
// multiples of 64 (check_gemm_shape). The tail skip is compiled into the
// row-grouped modes except dx, whose second copy of the K loop costs more
// registers than the skip saves.
template <int MODE, int ACT = kSwiGLU>
static void launch_mode(const GemmParams& p, int64_t R, hipStream_t stream) {
  if constexpr (MODE == kFwdGateUp || MODE == kFwdDown) {
    if constexpr (MODE == kFwdGateUp && ACT == kSwiGLU) {
      if (p.D >= 4096) {  // long contractions: 128-byte rows per stage, eight 64 x 64 waves
        launch_cfg<MODE, 8, 2, 4, 4, 3, true, 1, ACT, 64>(p, R, stream);
        return;
      }
      if (R >= 512 * (int64_t)p.E) {  // tall experts: 256 x 256 tiles, whole 128-byte rows
        launch_cfg<MODE, 8, 4, 4, 8, 2, true, 1, ACT, 64>(p, R, stream);
        return;
      }
    }
    if constexpr (MODE == kFwdGateUp && ACT == kOssGLU) {
      if (R >= 512 * (int64_t)p.E) {  // tall experts (gpt-oss-20b: 2048 rows per expert)
        launch_cfg<MODE, 8, 4, 4, 8, 2, true, 1, ACT, 64>(p, R, stream);
        return;
      }
    }
    if constexpr (MODE == kFwdDown && ACT == kSwiGLU) {
      // short experts with a long contraction (DSv3: H = 2048, 256 rows per expert):
      // gate_up's long-contraction tile (DSv3 down 2.72-2.74 -> 2.54-2.55 ms in the layer)
      if (p.H >= 2048 && R < 512 * (int64_t)p.E) {
        launch_cfg<MODE, 8, 2, 4, 4, 3, true, 1, ACT, 64>(p, R, stream);
        return;
      }
    }
    if constexpr (MODE == kFwdDown) {
      if (R >= 512 * (int64_t)p.E) {  // tall experts
        launch_cfg<MODE, 8, 4, 4, 8, 2, true, 1, ACT, 64>(p, R, stream);
        return;
      }
    }
    launch_cfg<MODE, 4, 2, 4, 8, 2, true, 2, ACT>(p, R, stream);
  } else if constexpr (MODE == kBwdDgu) {
    launch_cfg<MODE, 4, 2, 4, 8, 2, true, 2, ACT>(p, R, stream);
  } else if constexpr (MODE == kBwdDx) {
    if (p.D % 384 == 0) launch_cfg<MODE, 8, 2, 4, 6, 3, false, 1, ACT>(p, R, stream);
    else if (p.D % 512 == 0) launch_cfg<MODE, 8, 2, 4, 8, 3, false, 1, ACT>(p, R, stream);
    else launch_cfg<MODE, 4, 2, 4, 8, 2, false, 2, ACT>(p, R, stream);
  } else {
    launch_cfg<MODE, 8, 4, 4, 8, 3, false, 1, kSwiGLU>(p, R, stream);
  }
}

static int check_gemm_shape(int64_t R, int32_t E, int32_t D, int32_t H) {
  if (R < 0 || E < 1 || E > kGemmMaxE || D < 64 || H < 64) return kErrInvalidArgument;
  if (D % 64 || H % 64) return kErrUnsupportedShape;
  if (R >= (int64_t)INT32_MAX / 2) return kErrUnsupportedShape;
  return kOk;
}

}  // namespace moe

using namespace moe;

static int gemm_params(GemmParams& p, const int64_t* counts, int64_t n_rows, int32_t n_experts,
                       int32_t dim, int32_t hidden) {
  const int st = check_gemm_shape(n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (!counts) return kErrInvalidArgument;
  p = GemmParams{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.D = dim; p.H = hidden;
  p.w13_estride = (int64_t)hidden * dim;
  p.w13_rstride = dim;
  return kOk;
}

MOE_API int moe_grouped_gemm_gate_up(const uint16_t* x, const uint16_t* w1, const uint16_t* w3,
                                     const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                     int32_t dim, int32_t hidden, uint16_t* g, uint16_t* u,
                                     uint16_t* h, hipStream_t stream) {
  GemmParams p;
  int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!x || !w1 || !w3 || !g || !u || !h) return kErrInvalidArgument;
  p.x = x; p.w1 = w1; p.w3 = w3; p.out_g = g; p.out_u = u; p.out_h = h;
  launch_mode<kFwdGateUp>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_down(const uint16_t* h, const uint16_t* w2, const int64_t* counts,
                                  int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                  uint16_t* y, hipStream_t stream) {
  GemmParams p;
  int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!h || !w2 || !y) return kErrInvalidArgument;
  p.h = h; p.w2 = w2; p.out_y = y;
  launch_mode<kFwdDown>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_bwd_dgu(const uint16_t* dy, const uint16_t* w2, const uint16_t* g,
                                     const uint16_t* u, const int64_t* counts, int64_t n_rows,
                                     int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* dgu,
                                     hipStream_t stream) {
  GemmParams p;
  int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!dy || !w2 || !g || !u || !dgu) return kErrInvalidArgument;
  p.dy = dy; p.w2 = w2; p.g = g; p.u = u; p.out_dgu = dgu;
  launch_mode<kBwdDgu>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_bwd_dx(const uint16_t* dgu, const uint16_t* w1, const uint16_t* w3,
                                    const int64_t* counts, int64_t n_rows, int32_t n_experts,
                                    int32_t dim, int32_t hidden, uint16_t* dx, hipStream_t stream) {
  GemmParams p;
  int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!dgu || !w1 || !w3 || !dx) return kErrInvalidArgument;
  p.dgu = dgu; p.w1 = w1; p.w3 = w3; p.out_dx = dx;
  launch_mode<kBwdDx>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_bwd_dw13(const uint16_t* dgu, const uint16_t* x, const int64_t* counts,
                                      int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                      uint16_t* dw1, uint16_t* dw3, hipStream_t stream) {
  GemmParams p;
  int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (!dw1 || !dw3 || (n_rows > 0 && (!dgu || !x))) return kErrInvalidArgument;
  p.dgu = dgu; p.x = x; p.out_dw1 = dw1; p.out_dw3 = dw3;
  launch_mode<kBwdDw13>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_bwd_dw2(const uint16_t* dy, const uint16_t* h, const int64_t* counts,
                                     int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                     uint16_t* dw2, hipStream_t stream) {
  GemmParams p;
  int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  if (!dw2 || (n_rows > 0 && (!dy || !h))) return kErrInvalidArgument;
  p.dy = dy; p.h = h; p.out_dw2 = dw2;
  launch_mode<kBwdDw2>(p, n_rows, stream);
  return launch_status();
}

// The SwiGLU epilogues' pointwise arithmetic on its own: fp32 silu(g) and sigmoid(g)
// of bf16 g as gate_up and dgu compute them, so that tests can compare every bf16
// input with torch's. Each pair (2i, 2i + 1) takes the fast form when both lie in its
// range, as a piece of the epilogues does when it lies in it for every lane.
__global__ void __launch_bounds__(256) swiglu_pointwise_kernel(const uint16_t* __restrict__ g,
                                                               float* __restrict__ silu,
                                                               float* __restrict__ sig, int64_t n) {
  const int64_t i = 2 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
  if (i >= n) return;
  const bool two = i + 1 < n;
  const float g0 = bf2f(g[i]), g1 = two ? bf2f(g[i + 1]) : 0.0f;
  const bool fast = silu_fast_range(fminf(g0, g1), fmaxf(g0, g1));
  const float d0 = silu_den(g0), d1 = silu_den(g1);
  const SiluSig r0 = fast ? silu_sig<true>(g0, d0) : silu_sig<false>(g0, d0);
  const SiluSig r1 = fast ? silu_sig<true>(g1, d1) : silu_sig<false>(g1, d1);
  silu[i] = r0.silu;
  sig[i] = r0.sig;
  if (two) {
    silu[i + 1] = r1.silu;
    sig[i + 1] = r1.sig;
  }
}

MOE_API int moe_swiglu_pointwise_f32(const uint16_t* g, float* silu, float* sigmoid, int64_t n,
                                     hipStream_t stream) {
  if (n < 0) return kErrInvalidArgument;
  if (n == 0) return kOk;
  if (!g || !silu || !sigmoid) return kErrInvalidArgument;
  const int64_t blocks = ((n + 1) / 2 + 255) / 256;
  if (blocks > 0x7fffffff) return kErrInvalidArgument;
  swiglu_pointwise_kernel<<<(unsigned)blocks, 256, 0, stream>>>(g, silu, sigmoid, n);
  return launch_status();
}

MOE_API int moe_grouped_swiglu_fwd(const uint16_t* x, const uint16_t* w1, const uint16_t* w2,
                                   const uint16_t* w3, const int64_t* counts, int64_t n_rows,
                                   int32_t n_experts, int32_t dim, int32_t hidden, uint16_t* g,
                                   uint16_t* u, uint16_t* h, uint16_t* y, hipStream_t stream) {
  int st = moe_grouped_gemm_gate_up(x, w1, w3, counts, n_rows, n_experts, dim, hidden, g, u, h, stream);
  if (st) return st;
  return moe_grouped_gemm_down(h, w2, counts, n_rows, n_experts, dim, hidden, y, stream);
}

MOE_API int moe_grouped_swiglu_bwd(const uint16_t* dy, const uint16_t* x, const uint16_t* w1,
                                   const uint16_t* w2, const uint16_t* w3, const int64_t* counts,
                                   const uint16_t* g, const uint16_t* u, const uint16_t* h,
                                   int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                   uint16_t* dgu_workspace, uint16_t* dx, uint16_t* dw1,
                                   uint16_t* dw2, uint16_t* dw3, hipStream_t stream) {
  int st = moe_grouped_gemm_bwd_dgu(dy, w2, g, u, counts, n_rows, n_experts, dim, hidden,
                                    dgu_workspace, stream);
  if (st) return st;
  st = moe_grouped_gemm_bwd_dx(dgu_workspace, w1, w3, counts, n_rows, n_experts, dim, hidden, dx, stream);
  if (st) return st;
  st = moe_grouped_gemm_bwd_dw13(dgu_workspace, x, counts, n_rows, n_experts, dim, hidden, dw1, dw3, stream);
  if (st) return st;
  return moe_grouped_gemm_bwd_dw2(dy, h, counts, n_rows, n_experts, dim, hidden, dw2, stream);
}

// ---------------------------------------------------------------------------
// gpt-oss experts (torchtitan/models/gpt_oss/moe.py:92-122): mlp1_weight
// [E, 2H, D] with glu row 2j and linear row 2j + 1, mlp1_bias [E, 2H],
// mlp2_weight [E, D, H], mlp2_bias [E, D]; swiglu with alpha 1.702 and a
// clamp limit. The same kernels with interleaved w1 / w3 row strides and the
// biased, clamped epilogues; the saved g / u are the biased pre-clamp halves.
// ---------------------------------------------------------------------------

static constexpr float kOssAlpha = 1.702f;

static int oss_params(GemmParams& p, const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                      int32_t hidden, const uint16_t* mlp1) {
  const int st = gemm_params(p, counts, n_rows, n_experts, dim, hidden);
  if (st) return st;
  p.w1 = mlp1;
  p.w3 = mlp1 ? mlp1 + dim : nullptr;
  p.w13_estride = 2 * (int64_t)hidden * dim;
  p.w13_rstride = 2 * (int64_t)dim;
  p.alpha = kOssAlpha;
  return kOk;
}

static float bf16_round_host(float v) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  if ((u & 0x7f800000u) != 0x7f800000u) u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

MOE_API int moe_grouped_gemm_oss_gate_up(const uint16_t* x, const uint16_t* mlp1_weight, const uint16_t* mlp1_bias,
                                         const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                         int32_t hidden, float swiglu_limit, uint16_t* g, uint16_t* u, uint16_t* h,
                                         hipStream_t stream) {
  GemmParams p;
  int st = oss_params(p, counts, n_rows, n_experts, dim, hidden, mlp1_weight);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!x || !mlp1_weight || !mlp1_bias || !g || !u || !h) return kErrInvalidArgument;
  p.x = x; p.b1 = mlp1_bias; p.limit = bf16_round_host(swiglu_limit);
  p.out_g = g; p.out_u = u; p.out_h = h;
  launch_mode<kFwdGateUp, kOssGLU>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_oss_down(const uint16_t* h, const uint16_t* mlp2_weight, const uint16_t* mlp2_bias,
                                      const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                      int32_t hidden, uint16_t* y, hipStream_t stream) {
  GemmParams p;
  int st = oss_params(p, counts, n_rows, n_experts, dim, hidden, nullptr);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!h || !mlp2_weight || !mlp2_bias || !y) return kErrInvalidArgument;
  p.h = h; p.w2 = mlp2_weight; p.b2 = mlp2_bias; p.out_y = y;
  launch_mode<kFwdDown, kOssGLU>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_oss_bwd_dgu(const uint16_t* dy, const uint16_t* mlp2_weight, const uint16_t* g,
                                         const uint16_t* u, const int64_t* counts, int64_t n_rows,
                                         int32_t n_experts, int32_t dim, int32_t hidden, float swiglu_limit,
                                         uint16_t* dgu, hipStream_t stream) {
  GemmParams p;
  int st = oss_params(p, counts, n_rows, n_experts, dim, hidden, nullptr);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!dy || !mlp2_weight || !g || !u || !dgu) return kErrInvalidArgument;
  p.dy = dy; p.w2 = mlp2_weight; p.g = g; p.u = u; p.out_dgu = dgu; p.limit = bf16_round_host(swiglu_limit);
  launch_mode<kBwdDgu, kOssGLU>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_oss_bwd_dx(const uint16_t* dgu, const uint16_t* mlp1_weight, const int64_t* counts,
                                        int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                        uint16_t* dx, hipStream_t stream) {
  GemmParams p;
  int st = oss_params(p, counts, n_rows, n_experts, dim, hidden, mlp1_weight);
  if (st) return st;
  if (n_rows == 0) return kOk;
  if (!dgu || !mlp1_weight || !dx) return kErrInvalidArgument;
  p.dgu = dgu; p.out_dx = dx;
  launch_mode<kBwdDx, kOssGLU>(p, n_rows, stream);
  return launch_status();
}

MOE_API int moe_grouped_gemm_oss_bwd_dw1(const uint16_t* dgu, const uint16_t* x, const int64_t* counts,
                                         int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden,
                                         uint16_t* dmlp1_weight, hipStream_t stream) {
  GemmParams p;
  int st = oss_params(p, counts, n_rows, n_experts, dim, hidden, nullptr);
  if (st) return st;
  if (!dmlp1_weight || (n_rows > 0 && (!dgu || !x))) return kErrInvalidArgument;
  p.dgu = dgu; p.x = x; p.out_dw1 = dmlp1_weight; p.out_dw3 = dmlp1_weight + dim;
  launch_mode<kBwdDw13>(p, n_rows, stream);
  return launch_status();
}
