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
//  * 256 threads = 4 waves in 2 x 2; block tile BM x BN x BK (128 x 256 x 32);
//    wave tile 64 x 128 of v_mfma_f32_16x16x32_bf16 (fp32 accumulate); two
//    workgroups per CU.
//  * Two LDS stages. Stage k+1 is loaded from HBM into registers while stage k
//    feeds the MFMAs, then stored to the other LDS buffer; one barrier per K
//    step. The LDS tile is chunk-major (each 16-byte k-chunk of all rows is
//    contiguous, rows XOR-permuted inside 8-row groups), which on gfx950
//    measures free of bank conflicts for both the 16-byte fragment reads and
//    the 16-byte tile stores; a row-major tile costs ~4 conflict cycles per read.
//  * Operands that are contiguous along m/n in HBM (the weights in dgu/dx,
//    the token-major activations in dW) are transposed in registers while
//    staging: each thread loads KB k-rows of 8 contiguous elements and writes
//    8 LDS rows of KB elements.
//  * Persistent grid. Each workgroup derives the expert segments and
//    per-expert tile counts from num_tokens_per_expert in LDS (atomics-free
//    scan), so empty and heavily loaded experts need no host sync and no
//    padding. Workgroup ids are remapped so each XCD works on a contiguous
//    window of tiles (neighbouring tiles share an operand in its L2).
//  * The K loop runs in ascending k in steps of 32 and each output element is
//    rounded to bf16 once, at the points the reference's bf16 autograd rounds;
//    the outputs are bit-identical to torch._grouped_mm and its autograd on
//    this GPU.
#include "common.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmMaxE = 1024;
constexpr int kThreads = 256;

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
};

// LDS tile layout (measured conflict-free on gfx950 for 16-byte fragment reads
// of 16 consecutive rows and for 16-byte tile stores of 4 lanes per row):
// chunk-major, i.e. the 16-byte k-chunk kc of all ROWS rows is contiguous,
// with rows permuted inside each 8-row group by an XOR of the chunk index and
// the group index. Returns the element offset of (row r, chunk kc).
template <int ROWS>
__device__ __forceinline__ int lds_off(int r, int kc) {
  return (kc * ROWS + (r ^ (((2 * kc) ^ (r >> 3)) & 7))) * 8;
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

template <int MODE>
struct ModeTraits {
  static constexpr bool kRowGrouped = MODE <= kBwdDx;   // m = token rows of one expert
  static constexpr bool kPT = MODE >= kBwdDw13;          // P contiguous along m
  static constexpr bool kQT = MODE >= kBwdDgu;           // Q contiguous along n
};

// Interleave of the gate_up output columns: 16-column blocks alternate
// between g (w1) and u (w3), so a lane's SwiGLU operands sit in one wave.
__device__ __forceinline__ const uint16_t* gate_up_row(const GemmParams& p, int64_t e, int nt, int n, int BN) {
  const int blk = n >> 4;
  const int hc = nt * (BN / 2) + (blk >> 1) * 16 + (n & 15);
  return ((blk & 1) ? p.w3 : p.w1) + (e * p.H + hc) * (int64_t)p.D;
}

template <int MODE, int BM, int BN, int BK, int STAGES, int OCC, bool PD>
__global__ __launch_bounds__(kThreads, OCC) void grouped_gemm_kernel(GemmParams p) {
  using T = ModeTraits<MODE>;
  // PD: the K-contiguous P operand (token rows) bypasses LDS: each lane loads
  // its MFMA fragment (16 contiguous bytes of one row) straight from HBM.
  static_assert(!PD || (!T::kPT && BK == 32), "direct P fragments need K-contiguous P and BK = 32");
  constexpr int CPR = BK / 8;  // 16-byte chunks per LDS row
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  // staging shapes
  constexpr int PK_CH = BM * BK / 8 / kThreads;  // 16-byte chunks per thread, K-contiguous P
  constexpr int QK_CH = BN * BK / 8 / kThreads;
  constexpr int PT_KB = BM * BK / 8 / kThreads;  // k-rows per thread, m-contiguous P (8 m each)
  constexpr int QT_KB = BN * BK / 8 / kThreads;
  static_assert(PK_CH >= 1 && QK_CH >= 1, "tile too small for 256 threads");
  static_assert(!T::kPT || PT_KB == 2 || PT_KB == 4 || PT_KB == 8, "transposed P staging: 2, 4 or 8 k-rows");
  static_assert(!T::kQT || QT_KB == 2 || QT_KB == 4 || QT_KB == 8, "transposed Q staging: 2, 4 or 8 k-rows");
  static_assert(BK % 32 == 0 && (CPR == 4 || CPR == 8), "BK must be 32 or 64");

  constexpr int LDS_STAGES = STAGES == 1 ? 1 : 2;
  __shared__ __attribute__((aligned(16))) uint16_t sP[LDS_STAGES][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sQ[LDS_STAGES][BN * BK];
  __shared__ int s_seg[kGemmMaxE + 1];
  __shared__ int s_tile[kGemmMaxE + 1];
  __shared__ int s_tmp[8];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int E = p.E, D = p.D, H = p.H;

  int Ntot = 0, Kfix = 0, Mfix = 0;
  if (MODE == kFwdGateUp) { Ntot = 2 * H; Kfix = D; }
  if (MODE == kFwdDown) { Ntot = D; Kfix = H; }
  if (MODE == kBwdDgu) { Ntot = H; Kfix = D; }
  if (MODE == kBwdDx) { Ntot = D; Kfix = 2 * H; }
  if (MODE == kBwdDw13) { Ntot = D; Mfix = 2 * H; }
  if (MODE == kBwdDw2) { Ntot = H; Mfix = D; }
  const int NT = Ntot / BN;
  const int MT = T::kRowGrouped ? 0 : Mfix / BM;

  // ---- expert segments and tile table (LDS) ----
  {
    int cnt[4], tl[4], seg[4], tst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      const int64_t c = (e < E) ? p.counts[e] : 0;
      cnt[i] = c < 0 ? 0 : (c > p.R ? (int)p.R : (int)c);
    }
    {
      // clamp the running segment ends to R so inconsistent counts never read past the rows
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
      if (e < E) {
        s_seg[e] = seg[i];
        s_tile[e] = tst[i];
      }
    }
    if (tid == 0) {
      s_seg[E] = rtot;
      s_tile[E] = ttot;
    }
    __syncthreads();
  }
  const int total_tiles = s_tile[E];
  const int G = gridDim.x;
  const int lb = (G % 8 == 0) ? ((int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3)) : (int)blockIdx.x;

  for (int t = lb; t < total_tiles; t += G) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_tile[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int e = lo;
    const int64_t e64 = e;
    const int local = t - s_tile[e];
    const int seg0 = s_seg[e], seg1 = s_seg[e + 1];
    int mt, nt;
    if (T::kRowGrouped) {
      const int mtiles = (seg1 - seg0 + BM - 1) / BM;
      nt = local / mtiles;
      mt = local - nt * mtiles;
    } else {
      nt = local / MT;
      mt = local - nt * MT;
    }
    const int Ktot = T::kRowGrouped ? Kfix : (seg1 - seg0);
    const int nk = (Ktot + BK - 1) / BK;
    const int row0 = seg0 + mt * BM;  // first token row of a row-grouped tile

    struct Regs {
      uint4 p[PD ? TM : (T::kPT ? PT_KB : PK_CH)];
      uint4 q[T::kQT ? QT_KB : QK_CH];
    };
    Regs ra, rb;

    // ---- global -> registers for K step kt ----
    auto load_stage = [&](Regs& rr, int kt) {
      uint4* rp = rr.p;
      uint4* rq = rr.q;
      const int k0 = kt * BK;
      // P
      if constexpr (!T::kPT) {
        const uint16_t* pb;
        int ldp;
        if (MODE == kFwdGateUp) { pb = p.x; ldp = D; }
        else if (MODE == kFwdDown) { pb = p.h; ldp = H; }
        else if (MODE == kBwdDgu) { pb = p.dy; ldp = D; }
        else { pb = p.dgu; ldp = 2 * H; }
        if constexpr (PD) {
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            const int r = row0 + wm * WM + i * 16 + (lane & 15);
            rp[i] = (r < seg1) ? *(const uint4*)(pb + (int64_t)r * ldp + k0 + (lane >> 4) * 8) : make_uint4(0, 0, 0, 0);
          }
        } else
#pragma unroll
        for (int i = 0; i < PK_CH; ++i) {
          const int c = tid + i * kThreads;
          const int m = c / CPR, kc = c % CPR;
          const int r = row0 + m;
          rp[i] = (r < seg1) ? *(const uint4*)(pb + (int64_t)r * ldp + k0 + kc * 8) : make_uint4(0, 0, 0, 0);
        }
      } else {
        const uint16_t* pb = (MODE == kBwdDw13) ? p.dgu : p.dy;
        const int ldp = (MODE == kBwdDw13) ? 2 * H : D;
        constexpr int MB = BM / 8;
        const int mb = tid % MB, kb = tid / MB;
#pragma unroll
        for (int kk = 0; kk < PT_KB; ++kk) {
          const int r = seg0 + k0 + kb * PT_KB + kk;
          rp[kk] = (r < seg1) ? *(const uint4*)(pb + (int64_t)r * ldp + mt * BM + mb * 8) : make_uint4(0, 0, 0, 0);
        }
      }
      // Q
      if constexpr (!T::kQT) {
#pragma unroll
        for (int i = 0; i < QK_CH; ++i) {
          const int c = tid + i * kThreads;
          const int n = c / CPR, kc = c % CPR;
          const uint16_t* rowp = (MODE == kFwdGateUp) ? gate_up_row(p, e64, nt, n, BN)
                                                       : p.w2 + (e64 * D + nt * BN + n) * (int64_t)H;
          rq[i] = *(const uint4*)(rowp + k0 + kc * 8);
        }
      } else {
        constexpr int NB = BN / 8;
        const int nb = tid % NB, kb = tid / NB;
#pragma unroll
        for (int kk = 0; kk < QT_KB; ++kk) {
          const int k = k0 + kb * QT_KB + kk;
          const uint16_t* src;
          bool ok = true;
          if (MODE == kBwdDgu) {
            src = p.w2 + (e64 * D + k) * (int64_t)H;
          } else if (MODE == kBwdDx) {
            src = (k < H) ? p.w1 + (e64 * H + k) * (int64_t)D : p.w3 + (e64 * H + (k - H)) * (int64_t)D;
          } else {
            const int r = seg0 + k;
            ok = r < seg1;
            src = (MODE == kBwdDw13) ? p.x + (int64_t)r * D : p.h + (int64_t)r * H;
          }
          rq[kk] = ok ? *(const uint4*)(src + nt * BN + nb * 8) : make_uint4(0, 0, 0, 0);
        }
      }
    };

    // ---- registers -> LDS stage s ----
    auto store_stage = [&](const Regs& rr, int s) {
      const uint4* rp = rr.p;
      const uint4* rq = rr.q;
      uint16_t* dP = sP[s];
      uint16_t* dQ = sQ[s];
      if constexpr (PD) {
      } else if constexpr (!T::kPT) {
#pragma unroll
        for (int i = 0; i < PK_CH; ++i) {
          const int c = tid + i * kThreads;
          const int m = c / CPR, kc = c % CPR;
          *(uint4*)(dP + lds_off<BM>(m, kc)) = rp[i];
        }
      } else {
        constexpr int MB = BM / 8;
        const int mb = tid % MB, kb = tid / MB;
        const int kl = kb * PT_KB;  // first k of this thread's rows
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) {
          const int m = mb * 8 + mm;
          uint32_t o[PT_KB / 2];
#pragma unroll
          for (int j = 0; j < PT_KB / 2; ++j) {
            const uint32_t a = (&rp[2 * j].x)[mm >> 1], b = (&rp[2 * j + 1].x)[mm >> 1];
            o[j] = (mm & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
          }
          uint16_t* dst = dP + lds_off<BM>(m, kl >> 3) + (kl & 7);
          if constexpr (PT_KB == 8) *(uint4*)dst = make_uint4(o[0], o[1 % (PT_KB / 2)], o[2 % (PT_KB / 2)], o[3 % (PT_KB / 2)]);
          else if constexpr (PT_KB == 4) *(uint2*)dst = make_uint2(o[0], o[1 % (PT_KB / 2)]);
          else *(uint32_t*)dst = o[0];
        }
      }
      if constexpr (!T::kQT) {
#pragma unroll
        for (int i = 0; i < QK_CH; ++i) {
          const int c = tid + i * kThreads;
          const int n = c / CPR, kc = c % CPR;
          *(uint4*)(dQ + lds_off<BN>(n, kc)) = rq[i];
        }
      } else {
        constexpr int NB = BN / 8;
        const int nb = tid % NB, kb = tid / NB;
        const int kl = kb * QT_KB;
#pragma unroll
        for (int nn = 0; nn < 8; ++nn) {
          const int n = nb * 8 + nn;
          uint32_t o[QT_KB / 2];
#pragma unroll
          for (int j = 0; j < QT_KB / 2; ++j) {
            const uint32_t a = (&rq[2 * j].x)[nn >> 1], b = (&rq[2 * j + 1].x)[nn >> 1];
            o[j] = (nn & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
          }
          uint16_t* dst = dQ + lds_off<BN>(n, kl >> 3) + (kl & 7);
          if constexpr (QT_KB == 8) *(uint4*)dst = make_uint4(o[0], o[1 % (QT_KB / 2)], o[2 % (QT_KB / 2)], o[3 % (QT_KB / 2)]);
          else if constexpr (QT_KB == 4) *(uint2*)dst = make_uint2(o[0], o[1 % (QT_KB / 2)]);
          else *(uint32_t*)dst = o[0];
        }
      }
    };

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int ml = lane & 15, nq = (lane >> 4) * 4;
    // dx = dg.w1 + du.w3: the reference's autograd forms the two products as
    // separate bf16 GEMM outputs and adds them in bf16. The w1 half is rounded
    // and parked in the output rows (read back by the same lanes at the end).
    const int kt_half = (MODE == kBwdDx) ? H / BK : -1;

    auto park_dx_half = [&]() {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (r < seg1) {
            const int n = nt * BN + wn * WN + j * 16 + nq;
            *(uint2*)(p.out_dx + (int64_t)r * D + n) =
                make_uint2(pack_bf2(acc[i][j][0], acc[i][j][1]), pack_bf2(acc[i][j][2], acc[i][j][3]));
          }
          acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
    };

    auto compute_stage = [&](int s, const Regs& cur) {
      const uint16_t* cP = sP[s];
      const uint16_t* cQ = sQ[s];
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        const int kc = ks * 4 + (lane >> 4);
        bf16x8_t af[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = wm * WM + i * 16 + ml;
          if constexpr (PD) af[i] = __builtin_bit_cast(bf16x8_t, cur.p[i]);
          else af[i] = *(const bf16x8_t*)(cP + lds_off<BM>(m, kc));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = wn * WN + j * 16 + ml;
          const bf16x8_t bq = *(const bf16x8_t*)(cQ + lds_off<BN>(n, kc));
#pragma unroll
          for (int i = 0; i < TM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq, af[i], acc[i][j], 0, 0, 0);
        }
      }
    };

    if constexpr (STAGES == 3) {
      // two LDS stages and two register sets: stage kt+2 is in flight to
      // registers while stage kt feeds the MFMAs and stage kt+1 (loaded one
      // step earlier) is stored to the other LDS buffer; one barrier per step
      __syncthreads();  // the previous tile's last stage reads are done
      if (nk > 0) {
        load_stage(ra, 0);
        store_stage(ra, 0);
      }
      if (nk > 1) load_stage(ra, 1);
      __syncthreads();
      for (int kt = 0; kt < nk; kt += 2) {
        if (kt + 2 < nk) load_stage(rb, kt + 2);
        if (MODE == kBwdDx && kt == kt_half) park_dx_half();
        compute_stage(0, ra);
        if (kt + 1 < nk) store_stage(ra, 1);
        __syncthreads();
        if (kt + 1 >= nk) break;
        if (kt + 3 < nk) load_stage(ra, kt + 3);
        if (MODE == kBwdDx && kt + 1 == kt_half) park_dx_half();
        compute_stage(1, rb);
        if (kt + 2 < nk) store_stage(rb, 0);
        __syncthreads();
      }
    } else if constexpr (STAGES == 2) {
      // two LDS stages: stage kt+1 is loaded to registers during the MFMAs of
      // stage kt and stored to the other buffer; one barrier per K step
      __syncthreads();  // the previous tile's last stage reads are done
      if (nk > 0) {
        load_stage(ra, 0);
        store_stage(ra, 0);
      }
      __syncthreads();
      for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_stage(rb, kt + 1);
        if (MODE == kBwdDx && kt == kt_half) park_dx_half();
        compute_stage(cur, ra);
        if (kt + 1 < nk) store_stage(rb, cur ^ 1);
        if constexpr (PD) {
#pragma unroll
          for (int i = 0; i < TM; ++i) ra.p[i] = rb.p[i];
        }
        __syncthreads();
      }
    } else {
      // one LDS stage shared by two resident workgroups per CU: stage kt+1 is
      // loaded to registers during the MFMAs of stage kt
      if (nk > 0) load_stage(ra, 0);
      for (int kt = 0; kt < nk; ++kt) {
        __syncthreads();
        store_stage(ra, 0);
        __syncthreads();
        if (kt + 1 < nk) load_stage(ra, kt + 1);
        if (MODE == kBwdDx && kt == kt_half) park_dx_half();
        compute_stage(0, ra);
      }
    }

    // ---- epilogue: lane holds C[m = .. + ml][n = .. + nq + 0..3] ----
    if (MODE == kFwdGateUp) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
#pragma unroll
          for (int jj = 0; jj < TN / 2; ++jj) {
            const int hc = nt * (BN / 2) + wn * (WN / 2) + jj * 16 + nq;
            float gv[4], uv[4], hv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              gv[q] = round_bf(acc[i][2 * jj][q]);
              uv[q] = round_bf(acc[i][2 * jj + 1][q]);
              hv[q] = round_bf(silu_f(gv[q])) * uv[q];
            }
            const int64_t off = (int64_t)r * H + hc;
            *(uint2*)(p.out_g + off) = make_uint2(pack_bf2(gv[0], gv[1]), pack_bf2(gv[2], gv[3]));
            *(uint2*)(p.out_u + off) = make_uint2(pack_bf2(uv[0], uv[1]), pack_bf2(uv[2], uv[3]));
            *(uint2*)(p.out_h + off) = make_uint2(pack_bf2(hv[0], hv[1]), pack_bf2(hv[2], hv[3]));
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
          for (int j = 0; j < TN; ++j) {
            const int n = nt * BN + wn * WN + j * 16 + nq;
            uint16_t* dst = outp + (int64_t)r * D + n;
            float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            if (MODE == kBwdDx) {
              const uint2 pw = *(const uint2*)dst;
              v[0] = bf_lo(pw.x) + round_bf(v[0]);
              v[1] = bf_hi(pw.x) + round_bf(v[1]);
              v[2] = bf_lo(pw.y) + round_bf(v[2]);
              v[3] = bf_hi(pw.y) + round_bf(v[3]);
            }
            *(uint2*)dst = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
          }
        }
      }
    } else if (MODE == kBwdDgu) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int hh = nt * BN + wn * WN + j * 16 + nq;
            const int64_t off = (int64_t)r * H + hh;
            const uint2 gw = *(const uint2*)(p.g + off);
            const uint2 uw = *(const uint2*)(p.u + off);
            const float gv[4] = {bf_lo(gw.x), bf_hi(gw.x), bf_lo(gw.y), bf_hi(gw.y)};
            const float uv[4] = {bf_lo(uw.x), bf_hi(uw.x), bf_lo(uw.y), bf_hi(uw.y)};
            float dg[4], du[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float dh = round_bf(acc[i][j][q]);
              const float sl = round_bf(silu_f(gv[q]));         // saved silu(g) (bf16)
              const float dsl = round_bf(dh * uv[q]);           // d silu(g)
              du[q] = dh * sl;                                  // d u
              const float sg = 1.0f / (1.0f + expf(-gv[q]));
              dg[q] = dsl * sg * (1.0f + gv[q] * (1.0f - sg));  // silu backward
            }
            const int64_t o2 = (int64_t)r * (2 * H) + hh;
            *(uint2*)(p.out_dgu + o2) = make_uint2(pack_bf2(dg[0], dg[1]), pack_bf2(dg[2], dg[3]));
            *(uint2*)(p.out_dgu + o2 + H) = make_uint2(pack_bf2(du[0], du[1]), pack_bf2(du[2], du[3]));
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = mt * BM + wm * WM + i * 16 + ml;
        uint16_t* rowp;
        if (MODE == kBwdDw13)
          rowp = (m < H) ? p.out_dw1 + (e64 * H + m) * (int64_t)D : p.out_dw3 + (e64 * H + (m - H)) * (int64_t)D;
        else
          rowp = p.out_dw2 + (e64 * D + m) * (int64_t)H;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = nt * BN + wn * WN + j * 16 + nq;
          *(uint2*)(rowp + n) =
              make_uint2(pack_bf2(acc[i][j][0], acc[i][j][1]), pack_bf2(acc[i][j][2], acc[i][j][3]));
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

// Tile shape per mode (BM x BN x BK, LDS stages). D and H are multiples of 256
// (check_gemm_shape), so every BM and BN here divides the fixed dimensions.
template <int MODE> struct Tile { static constexpr int BM = 128, BN = 256, BK = 32, STAGES = 2, OCC = 2; };

static int persistent_grid(int64_t max_tiles, int per_cu) {
  int64_t g = (int64_t)cu_count() * per_cu;
  if (g > max_tiles) g = max_tiles;
  if (g >= 8) g -= g % 8;
  return (int)(g < 1 ? 1 : g);
}

template <int MODE, int BM, int BN, int BK, int ST, int OCC, bool PD>
static void launch_cfg(const GemmParams& p, int64_t R, hipStream_t stream) {
  int64_t max_tiles;
  if (MODE == kFwdGateUp) max_tiles = (R / BM + p.E) * (2 * p.H / BN);
  else if (MODE == kFwdDown || MODE == kBwdDx) max_tiles = (R / BM + p.E) * (p.D / BN);
  else if (MODE == kBwdDgu) max_tiles = (R / BM + p.E) * (p.H / BN);
  else if (MODE == kBwdDw13) max_tiles = (int64_t)p.E * (2 * p.H / BM) * (p.D / BN);
  else max_tiles = (int64_t)p.E * (p.D / BM) * (p.H / BN);
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE, BM, BN, BK, ST, OCC, PD>), dim3(persistent_grid(max_tiles, OCC)),
                     dim3(kThreads), 0, stream, p);
}

template <int MODE>
static void launch_mode(const GemmParams& p, int64_t R, hipStream_t stream) {
  using C = Tile<MODE>;
  launch_cfg<MODE, C::BM, C::BN, C::BK, C::STAGES, C::OCC, false>(p, R, stream);
}

static int check_gemm_shape(int64_t R, int32_t E, int32_t D, int32_t H) {
  if (R < 0 || E < 1 || E > kGemmMaxE || D < 256 || H < 256) return kErrInvalidArgument;
  if (D % 256 || H % 256) return kErrUnsupportedShape;
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
