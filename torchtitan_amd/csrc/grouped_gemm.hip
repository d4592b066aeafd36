// Persistent grouped GEMMs for the SwiGLU experts on MI355X (bf16 MFMA).
//
// Replaces the three torch._grouped_mm calls of
// torchtitan/models/common/moe.py:53-70 (_run_experts_grouped_mm) and their
// autograd. Expert e owns the rows [start_e, start_e + count_e) of the routed
// activations (start = exclusive cumsum of num_tokens_per_expert, moe.py:60).
//
// Design:
//  * One kernel template, six problem modes (forward gate/up, forward down,
//    backward dh, dx, dW1/dW3, dW2). Every mode is a C[m][n] = sum_k P[m][k] Q[n][k]
//    with both operands staged in LDS K-major, so the inner loop is always
//    ds_read_b128 + v_mfma_f32_16x16x32_bf16. Operands that are contiguous
//    along M/N in HBM (weights read transposed in backward, token-major
//    activations in dW) are transposed in registers while staging.
//  * Workgroup tile BM x 256 x 64, 4 waves in 2x2, each wave (BM/2) x 128.
//  * Persistent grid (2 workgroups per CU); each workgroup derives the expert
//    segment starts and per-expert tile counts from num_tokens_per_expert in
//    LDS (atomics-free scan), so empty and heavily loaded experts need no host
//    sync and no padding. Tile ids are remapped so that concurrently running
//    tiles of one expert land on one XCD and share its L2.
//  * Epilogues: gate/up pairs are interleaved in 16-column blocks so SwiGLU
//    (and its backward) is lane-local; results are rounded to bf16 at the
//    points the reference's bf16 autograd rounds them.
#include "common.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmBK = 64;
constexpr int kGemmBN = 256;
constexpr int kGemmMaxE = 1024;

enum GemmMode : int {
  kFwdGateUp = 0,  // [g|u][r, :] = X[r] . {w1,w3}[e]^T ; h = silu(g) * u
  kFwdDown = 1,    // y[r] = h[r] . w2[e]^T
  kBwdDh = 2,      // dh[r] = dy[r] . w2[e] ; -> (dg, du) via SwiGLU backward
  kBwdDx = 3,      // dx[r] = dg[r] . w1[e] + du[r] . w3[e]
  kBwdDw13 = 4,    // dw1[e] = dg_e^T . X_e ; dw3[e] = du_e^T . X_e
  kBwdDw2 = 5,     // dw2[e] = dy_e^T . h_e
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

__device__ __forceinline__ int lds_swz(int row) { return (row ^ (row >> 3)) & 7; }

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

template <int MODE, int BM>
__global__ __launch_bounds__(256, 2) void grouped_gemm_kernel(GemmParams p) {
  constexpr int BN = kGemmBN, BK = kGemmBK;
  constexpr bool kRowGrouped = (MODE <= kBwdDx);
  constexpr bool kBKmajor = (MODE == kFwdGateUp || MODE == kFwdDown);
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int ACH = BM / 32;  // 16-byte staging registers per thread for A
  constexpr int BCH = BN / 32;  // ... for B

  __shared__ __attribute__((aligned(16))) uint16_t sA[BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[BN * BK];
  __shared__ int s_seg[kGemmMaxE + 1];
  __shared__ int s_tile[kGemmMaxE + 1];
  __shared__ int s_tmp[8];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int E = p.E, D = p.D, H = p.H;

  // Problem extents per mode: N (output columns), fixed K, fixed M (dW only).
  int Ntot, Kfix = 0, Mfix = 0;
  if (MODE == kFwdGateUp) { Ntot = 2 * H; Kfix = D; }
  if (MODE == kFwdDown) { Ntot = D; Kfix = H; }
  if (MODE == kBwdDh) { Ntot = H; Kfix = D; }
  if (MODE == kBwdDx) { Ntot = D; Kfix = 2 * H; }
  if (MODE == kBwdDw13) { Ntot = D; Mfix = 2 * H; }
  if (MODE == kBwdDw2) { Ntot = H; Mfix = D; }
  const int NT = Ntot / BN;
  const int MT = kRowGrouped ? 0 : Mfix / BM;

  {
    int cnt[4], tl[4], seg[4], tst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid * 4 + i;
      const int64_t c = (e < E) ? p.counts[e] : 0;
      cnt[i] = c < 0 ? 0 : (c > p.R ? (int)p.R : (int)c);
    }
    // clamp the running segment ends to R so inconsistent counts never read past the rows
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
      tl[i] = (e < E) ? (kRowGrouped ? ((cnt[i] + BM - 1) / BM) * NT : MT * NT) : 0;
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
    const int local = t - s_tile[e];
    const int seg0 = s_seg[e], seg1 = s_seg[e + 1];
    int mt, nt;
    if (kRowGrouped) {
      const int mtiles = (seg1 - seg0 + BM - 1) / BM;
      nt = local / mtiles;
      mt = local - nt * mtiles;
    } else {
      nt = local / MT;
      mt = local - nt * MT;
    }
    const int Ktot = kRowGrouped ? Kfix : (seg1 - seg0);
    const int nk = (Ktot + BK - 1) / BK;
    const int row0 = seg0 + mt * BM;  // first token row of a row-grouped tile
    const int64_t e64 = e;

    uint4 ra[ACH], rb[BCH];

    // ---- global -> registers ------------------------------------------------
    auto load_tile = [&](int kt) {
      const int k0 = kt * BK;
      if (kRowGrouped) {
        const uint16_t* abase;
        int lda;
        if (MODE == kFwdGateUp || MODE == kBwdDh) { abase = (MODE == kFwdGateUp) ? p.x : p.dy; lda = D; }
        else if (MODE == kFwdDown) { abase = p.h; lda = H; }
        else { abase = p.dgu; lda = 2 * H; }
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
          const int c = tid + i * 256;
          const int m = c >> 3, kc = c & 7;
          const int r = row0 + m;
          ra[i] = (r < seg1) ? *(const uint4*)(abase + (int64_t)r * lda + k0 + kc * 8) : make_uint4(0, 0, 0, 0);
        }
      } else {
        // A[m][k] with k = token row, contiguous along m
        const uint16_t* abase = (MODE == kBwdDw13) ? p.dgu : p.dy;
        const int lda = (MODE == kBwdDw13) ? 2 * H : D;
        constexpr int KB = BM / 32;
        constexpr int MB = BM / 8;
        const int mnb = tid % MB, kb = tid / MB;
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
          const int r = seg0 + k0 + kb * KB + kk;
          ra[kk] = (r < seg1) ? *(const uint4*)(abase + (int64_t)r * lda + mt * BM + mnb * 8) : make_uint4(0, 0, 0, 0);
        }
      }
      if (kBKmajor) {
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
          const int c = tid + i * 256;
          const int n = c >> 3, kc = c & 7;
          const uint16_t* rowp;
          if (MODE == kFwdGateUp) {
            const int blk = n >> 4;
            const int hc = nt * 128 + (blk >> 1) * 16 + (n & 15);
            rowp = ((blk & 1) ? p.w3 : p.w1) + (e64 * H + hc) * D;
          } else {
            rowp = p.w2 + (e64 * D + nt * BN + n) * H;
          }
          rb[i] = *(const uint4*)(rowp + k0 + kc * 8);
        }
      } else {
        // B[n][k] contiguous along n: one 8(k) x 8(n) block per thread
        const int nb8 = tid & 31, kb = tid >> 5;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int k = k0 + kb * 8 + kk;
          const uint16_t* src = nullptr;
          bool ok = true;
          if (MODE == kBwdDh) {
            src = p.w2 + (e64 * D + k) * H;
          } else if (MODE == kBwdDx) {
            src = (k < H) ? p.w1 + (e64 * H + k) * D : p.w3 + (e64 * H + (k - H)) * D;
          } else {
            const int r = seg0 + k;
            ok = r < seg1;
            src = (MODE == kBwdDw13) ? p.x + (int64_t)r * D : p.h + (int64_t)r * H;
          }
          rb[kk] = ok ? *(const uint4*)(src + nt * BN + nb8 * 8) : make_uint4(0, 0, 0, 0);
        }
      }
    };

    // ---- registers -> LDS (K-major, 16-byte chunks XOR-swizzled per row) ----
    auto store_tile = [&]() {
      if (kRowGrouped) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
          const int c = tid + i * 256;
          const int m = c >> 3, kc = c & 7;
          *(uint4*)(sA + m * BK + ((kc ^ lds_swz(m)) << 3)) = ra[i];
        }
      } else {
        constexpr int KB = BM / 32;  // 4 k-values per thread (BM = 128)
        constexpr int MB = BM / 8;
        const int mnb = tid % MB, kb = tid / MB;
        const int kl = kb * KB;
        uint32_t in[KB][4];
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
          in[kk][0] = ra[kk].x; in[kk][1] = ra[kk].y; in[kk][2] = ra[kk].z; in[kk][3] = ra[kk].w;
        }
#pragma unroll
        for (int mm = 0; mm < 8; ++mm) {
          const int m = mnb * 8 + mm;
          uint32_t o[KB / 2];
#pragma unroll
          for (int j = 0; j < KB / 2; ++j) {
            const uint32_t a = in[2 * j][mm >> 1], b = in[2 * j + 1][mm >> 1];
            o[j] = (mm & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
          }
          uint16_t* dst = sA + m * BK + (((kl >> 3) ^ lds_swz(m)) << 3) + (kl & 7);
          if (KB == 8) *(uint4*)dst = make_uint4(o[0], o[1 % (KB / 2)], o[2 % (KB / 2)], o[3 % (KB / 2)]);
          else *(uint2*)dst = make_uint2(o[0], o[1 % (KB / 2)]);
        }
      }
      if (kBKmajor) {
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
          const int c = tid + i * 256;
          const int n = c >> 3, kc = c & 7;
          *(uint4*)(sB + n * BK + ((kc ^ lds_swz(n)) << 3)) = rb[i];
        }
      } else {
        const int nb8 = tid & 31, kb = tid >> 5;
        const int kl = kb * 8;
#pragma unroll
        for (int nn = 0; nn < 8; ++nn) {
          const int n = nb8 * 8 + nn;
          uint32_t o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t a = (&rb[2 * j].x)[nn >> 1], b = (&rb[2 * j + 1].x)[nn >> 1];
            o[j] = (nn & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
          }
          *(uint4*)(sB + n * BK + (((kl >> 3) ^ lds_swz(n)) << 3)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    };

    f32x4_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // dx = dg.w1 + du.w3: the reference's autograd forms the two products as
    // separate bf16 GEMM outputs and adds them in bf16, so the w1 half of the
    // reduction is rounded and held (packed bf16) when the w3 half starts.
    uint2 part[MODE == kBwdDx ? TM : 1][MODE == kBwdDx ? TN : 1];
    const int kt_half = (MODE == kBwdDx) ? H / BK : -1;

    if (nk > 0) load_tile(0);
    for (int kt = 0; kt < nk; ++kt) {
      if (MODE == kBwdDx && kt == kt_half) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            part[i][j] = make_uint2(pack_bf2(acc[i][j][0], acc[i][j][1]), pack_bf2(acc[i][j][2], acc[i][j][3]));
            acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
      }
      __syncthreads();
      store_tile();
      __syncthreads();
      if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        const int kc = ks * 4 + (lane >> 4);
        bf16x8_t af[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = wm * WM + i * 16 + (lane & 15);
          af[i] = *(const bf16x8_t*)(sA + m * BK + ((kc ^ lds_swz(m)) << 3));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = wn * WN + j * 16 + (lane & 15);
          const bf16x8_t bfr = *(const bf16x8_t*)(sB + n * BK + ((kc ^ lds_swz(n)) << 3));
#pragma unroll
          for (int i = 0; i < TM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr, af[i], acc[i][j], 0, 0, 0);
        }
      }
    }

    // ---- epilogue: lane holds C[m = .. + (lane&15)][n = .. + 4*(lane>>4) + 0..3] ----
    const int ml = lane & 15, nq = (lane >> 4) * 4;
    if (MODE == kFwdGateUp) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = row0 + wm * WM + i * 16 + ml;
        if (r < seg1) {
#pragma unroll
          for (int jj = 0; jj < TN / 2; ++jj) {
            const int hc = nt * 128 + wn * 64 + jj * 16 + nq;
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
            float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            if (MODE == kBwdDx) {
              const uint2 pw = part[i % (MODE == kBwdDx ? TM : 1)][j % (MODE == kBwdDx ? TN : 1)];
              v[0] = bf_lo(pw.x) + round_bf(v[0]);
              v[1] = bf_hi(pw.x) + round_bf(v[1]);
              v[2] = bf_lo(pw.y) + round_bf(v[2]);
              v[3] = bf_hi(pw.y) + round_bf(v[3]);
            }
            *(uint2*)(outp + (int64_t)r * D + n) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
          }
        }
      }
    } else if (MODE == kBwdDh) {
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
              const float sl = round_bf(silu_f(gv[q]));        // saved silu(g) (bf16)
              const float dsl = round_bf(dh * uv[q]);          // d silu(g)
              du[q] = dh * sl;                                 // d u
              const float sg = 1.0f / (1.0f + expf(-gv[q]));
              dg[q] = dsl * sg * (1.0f + gv[q] * (1.0f - sg)); // silu backward
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
        int ldo;
        if (MODE == kBwdDw13) {
          rowp = (m < H) ? p.out_dw1 + (e64 * H + m) * D : p.out_dw3 + (e64 * H + (m - H)) * D;
          ldo = D;
        } else {
          rowp = p.out_dw2 + (e64 * D + m) * H;
          ldo = H;
        }
        (void)ldo;
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

constexpr int kBM = 128;

static int persistent_grid(int64_t max_tiles) {
  int64_t g = (int64_t)cu_count() * 2;
  if (g > max_tiles) g = max_tiles;
  if (g >= 8) g -= g % 8;
  return (int)(g < 1 ? 1 : g);
}

template <int MODE>
static void launch_mode(const GemmParams& p, int64_t R, hipStream_t stream) {
  int64_t max_tiles;
  if (MODE == kFwdGateUp) max_tiles = (R / kBM + p.E) * (2 * p.H / kGemmBN);
  else if (MODE == kFwdDown || MODE == kBwdDx) max_tiles = (R / kBM + p.E) * (p.D / kGemmBN);
  else if (MODE == kBwdDh) max_tiles = (R / kBM + p.E) * (p.H / kGemmBN);
  else if (MODE == kBwdDw13) max_tiles = (int64_t)p.E * (2 * p.H / kBM) * (p.D / kGemmBN);
  else max_tiles = (int64_t)p.E * (p.D / kBM) * (p.H / kGemmBN);
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE, kBM>), dim3(persistent_grid(max_tiles)), dim3(256), 0,
                     stream, p);
}

static int check_gemm_shape(int64_t R, int32_t E, int32_t D, int32_t H) {
  if (R < 0 || E < 1 || E > kGemmMaxE || D < kGemmBN || H < kGemmBN) return kErrInvalidArgument;
  if (D % kGemmBN || H % kGemmBN) return kErrUnsupportedShape;
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
  launch_mode<kBwdDh>(p, n_rows, stream);
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
