// fp32 grouped GEMMs for the MoE experts in fp32 on MI355X (gfx950).
//
// The reference's readability path _run_experts_for_loop
// (torchtitan/models/common/moe.py:24-50) multiplies each expert's token
// segment in the input dtype: for fp32 models every product and sum is fp32.
// These kernels do the same arithmetic for all experts in one launch per GEMM,
// on v_mfma_f32_16x16x4f32 (fp32 operands, fp32 accumulation), with the
// SwiGLU of :41-43 and its autograd fused into the epilogues:
//   gate_up  g = x w1^T, u = x w3^T, h = silu(g) * u        (fp32 each)
//   down     y = h w2^T
//   bwd_dgu  dh = dy w2; du = dh * silu(g); dg = silu'(g) * (dh * u)
//   bwd_dx   dx = dg w1 + du w3
//   bwd_dw   out[e] = a_e^T b_e over expert e's rows (dw1, dw3, dw2)
//
// Tiles: 64 x 64 outputs per 256-thread workgroup, 16 of k per LDS stage, each
// wave a 32 x 32 quarter as 2 x 2 MFMA tiles. Operands are staged k-major in
// LDS (rows padded to 80 floats, so the 16-lane column reads of one k-row and
// the 64-lane scalar stores of one k-row are both free of bank conflicts).
// The next stage is loaded into registers while the current one computes.
// Row-grouped modes map blockIdx.x to (expert, 64-row tile) from a scan of the
// counts in LDS, so no host sync or padding is needed; surplus blocks exit.
#include "common.h"

namespace moe {
namespace f32g {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxE = 1024;
constexpr int BM = 64, BN = 64, BK = 16;
constexpr int LDS_ROW = 80;  // floats per k-row of a staged tile

enum Mode : int { kGateUp = 0, kDown = 1, kDgu = 2, kDx = 3, kDw = 4 };

struct Params {
  const int64_t* counts;
  int64_t R;
  int E;
  int N, K;        // row modes: N output columns, K contraction; dW: M = K (a's columns), N (b's columns)
  const float* a;  // row operand [R, K] (dW: [R, M])
  const float* a2; // second row operand (dx: du)
  const float* b;  // NT: [E, N, K]; NN: [E, K, N]; dW: [R, N]
  const float* b2; // second weight (gate_up: w3; dx: w3)
  const float* g;  // dgu: saved g, u [R, N]
  const float* u;
  float* o0;
  float* o1;
  float* o2;
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// expert e's segment: rows [start, start + count) clamped to R; tiles of 64 rows
struct Seg {
  int64_t start;
  int count;
  int tile;  // first 64-row tile of the expert (row modes)
};

// Which expert (and 64-row tile within it) block `bx` computes; e = -1 when bx
// is past the last tile. Every thread of the block must call it.
__device__ __forceinline__ void find_tile(const Params& p, int bx, int* s_tmp, int* s_out, int& e, Seg& seg,
                                          int& mt) {
  int cnt[4], tiles[4], st[4], tst[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ee = threadIdx.x * 4 + i;
    const int64_t c = ee < p.E ? p.counts[ee] : 0;
    cnt[i] = c < 0 ? 0 : (int)(c > p.R ? p.R : c);
  }
  block_exclusive_scan4(cnt, st, s_tmp);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // clamp the segment to R (counts that sum past R are cut at R)
    const int64_t room = p.R - st[i];
    cnt[i] = room <= 0 ? 0 : (cnt[i] > room ? (int)room : cnt[i]);
    tiles[i] = (cnt[i] + BM - 1) / BM;
  }
  block_exclusive_scan4(tiles, tst, s_tmp);
  if (threadIdx.x == 0) s_out[0] = -1;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ee = threadIdx.x * 4 + i;
    if (ee < p.E && tiles[i] > 0 && bx >= tst[i] && bx < tst[i] + tiles[i]) {
      s_out[0] = ee;
      s_out[1] = st[i];
      s_out[2] = cnt[i];
      s_out[3] = tst[i];
    }
  }
  __syncthreads();
  e = s_out[0];
  seg.start = s_out[1];
  seg.count = s_out[2];
  seg.tile = s_out[3];
  mt = bx - seg.tile;
}

// dW: start and count of expert e's rows
__device__ __forceinline__ void find_segment(const Params& p, int e, int* s_tmp, int* s_out, Seg& seg) {
  int cnt[4], st[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ee = threadIdx.x * 4 + i;
    const int64_t c = ee < p.E ? p.counts[ee] : 0;
    cnt[i] = c < 0 ? 0 : (int)(c > p.R ? p.R : c);
  }
  block_exclusive_scan4(cnt, st, s_tmp);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (threadIdx.x * 4 + i == e) {
      const int64_t room = p.R - st[i];
      s_out[0] = st[i];
      s_out[1] = room <= 0 ? 0 : (cnt[i] > room ? (int)room : cnt[i]);
    }
  }
  __syncthreads();
  seg.start = s_out[0];
  seg.count = s_out[1];
  seg.tile = 0;
}

// Staging of one 16-k slice.
//  rows operand [rows, K] (k contiguous), 64 rows: thread t holds row t % 64,
//    k (t / 64) * 4 .. + 3 (a 16-byte load) and stores them as 4 k-rows.
//  k-rows operand [k, cols] (cols contiguous), 64 cols: thread t holds k-row
//    t / 16, cols (t % 16) * 4 .. + 3, stored as one 16-byte LDS write.
__device__ __forceinline__ float4 load_rows(const float* base, int64_t ld, int row, int nrows, int k) {
  if (row >= nrows) return make_float4(0.f, 0.f, 0.f, 0.f);
  return *(const float4*)(base + (int64_t)row * ld + k);
}
__device__ __forceinline__ void store_rows(float* tile, const float4& v) {
  const int r = threadIdx.x & 63, k = (threadIdx.x >> 6) * 4;
  tile[(k + 0) * LDS_ROW + r] = v.x;
  tile[(k + 1) * LDS_ROW + r] = v.y;
  tile[(k + 2) * LDS_ROW + r] = v.z;
  tile[(k + 3) * LDS_ROW + r] = v.w;
}
__device__ __forceinline__ float4 load_krows(const float* base, int64_t ld, int krow, int nk) {
  if (krow >= nk) return make_float4(0.f, 0.f, 0.f, 0.f);
  return *(const float4*)(base + (int64_t)krow * ld + (threadIdx.x & 15) * 4);
}
__device__ __forceinline__ void store_krows(float* tile, const float4& v) {
  *(float4*)(tile + (threadIdx.x >> 4) * LDS_ROW + (threadIdx.x & 15) * 4) = v;
}

// One 16-k slice of MFMAs for this wave's 32 x 32 quarter.
__device__ __forceinline__ void mma_slice(const float* sa, const float* sb, int wm, int wn, int lane,
                                          f32x4_t (&acc)[2][2]) {
#pragma unroll
  for (int ks = 0; ks < BK; ks += 4) {
    const int k = ks + (lane >> 4);
    float av[2], bv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) av[i] = sa[k * LDS_ROW + 32 * wm + 16 * i + (lane & 15)];
#pragma unroll
    for (int j = 0; j < 2; ++j) bv[j] = sb[k * LDS_ROW + 32 * wn + 16 * j + (lane & 15)];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
  }
}

// Row-grouped modes: 64 rows of one expert x 64 output columns.
template <int MODE>
__global__ __launch_bounds__(256) void rows_kernel(Params p) {
  constexpr bool kTwoB = MODE == kGateUp;  // two weights into two accumulator sets
  constexpr bool kNT = MODE == kGateUp || MODE == kDown;  // weights [E, N, K]; else [E, K, N]
  __shared__ __attribute__((aligned(16))) float sA[BK * LDS_ROW];
  __shared__ __attribute__((aligned(16))) float sB[BK * LDS_ROW];
  __shared__ __attribute__((aligned(16))) float sB2[kTwoB ? BK * LDS_ROW : 4];
  __shared__ int s_tmp[8];
  __shared__ int s_out[4];
  int e, mt;
  Seg seg;
  find_tile(p, blockIdx.x, s_tmp, s_out, e, seg, mt);
  if (e < 0) return;
  const int n0 = blockIdx.y * BN;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
  const int64_t row0 = seg.start + (int64_t)mt * BM;
  const int nrows = seg.count - mt * BM < BM ? seg.count - mt * BM : BM;

  f32x4_t acc[2][2], acc2[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      acc2[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

  // weight slices for this block: NT [E, N, K] rows n0.. (k contiguous);
  // NN [E, K, N] k-rows with columns n0..
  const int phases = MODE == kDx ? 2 : 1;
  for (int ph = 0; ph < phases; ++ph) {
    const float* A = (ph == 0 ? p.a : p.a2) + row0 * p.K;
    const float* Bw = (ph == 0 ? p.b : p.b2) + (int64_t)e * p.N * p.K;
    const float* B2w = kTwoB ? p.b2 + (int64_t)e * p.N * p.K : nullptr;
    const int ar = threadIdx.x & 63, ak = (threadIdx.x >> 6) * 4;
    float4 ra, rb, rb2;
    auto fetch = [&](int k0) {
      ra = load_rows(A, p.K, ar, nrows, k0 + ak);
      if (kNT) {
        rb = load_rows(Bw + (int64_t)n0 * p.K, p.K, ar, BN, k0 + ak);
        if (kTwoB) rb2 = load_rows(B2w + (int64_t)n0 * p.K, p.K, ar, BN, k0 + ak);
      } else {
        rb = load_krows(Bw + (int64_t)k0 * p.N + n0, p.N, threadIdx.x >> 4, BK);
      }
    };
    fetch(0);
    for (int k0 = 0; k0 < p.K; k0 += BK) {
      __syncthreads();  // the previous slice's reads are done
      store_rows(sA, ra);
      if (kNT) {
        store_rows(sB, rb);
        if (kTwoB) store_rows(sB2, rb2);
      } else {
        store_krows(sB, rb);
      }
      __syncthreads();
      if (k0 + BK < p.K) fetch(k0 + BK);
      mma_slice(sA, sB, wm, wn, lane, acc);
      if (kTwoB) mma_slice(sA, sB2, wm, wn, lane, acc2);
    }
  }

  // epilogue: lane holds rows 4 (lane / 16) + v of each 16 x 16 tile, column lane % 16
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int lr = 32 * wm + 16 * i + 4 * (lane >> 4) + v;
        if (lr >= nrows) continue;
        const int64_t r = row0 + lr;
        const int64_t o = r * p.N + n0 + 32 * wn + 16 * j + (lane & 15);
        const float c = acc[i][j][v];
        if (MODE == kGateUp) {
          const float uu = acc2[i][j][v];
          p.o0[o] = c;
          p.o1[o] = uu;
          p.o2[o] = silu_f(c) * uu;
        } else if (MODE == kDgu) {
          const float gg = p.g[o], uu = p.u[o];
          const float sig = 1.0f / (1.0f + expf(-gg));
          p.o1[o] = c * silu_f(gg);                               // du = dh * silu(g)
          p.o0[o] = (c * uu) * (sig * (1.0f + gg * (1.0f - sig)));  // dg = silu'(g) (dh u)
        } else {
          p.o0[o] = c;
        }
      }
}

// Weight gradients: out[e][m][n] = sum over expert e's rows r of a[r][m] b[r][n].
__global__ __launch_bounds__(256) void dw_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float sA[BK * LDS_ROW];
  __shared__ __attribute__((aligned(16))) float sB[BK * LDS_ROW];
  __shared__ int s_tmp[8];
  __shared__ int s_out[2];
  const int e = blockIdx.x;
  Seg seg;
  find_segment(p, e, s_tmp, s_out, seg);
  const int M = p.K, N = p.N;
  const int ntn = N / BN;
  const int m0 = (blockIdx.y / ntn) * BM, n0 = (blockIdx.y % ntn) * BN;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const float* A = p.a + seg.start * M + m0;
  const float* B = p.b + seg.start * N + n0;
  float4 ra, rb;
  auto fetch = [&](int k0) {
    ra = load_krows(A + (int64_t)k0 * M, M, threadIdx.x >> 4, seg.count - k0);
    rb = load_krows(B + (int64_t)k0 * N, N, threadIdx.x >> 4, seg.count - k0);
  };
  if (seg.count > 0) fetch(0);
  for (int k0 = 0; k0 < seg.count; k0 += BK) {
    __syncthreads();
    store_krows(sA, ra);
    store_krows(sB, rb);
    __syncthreads();
    if (k0 + BK < seg.count) fetch(k0 + BK);
    mma_slice(sA, sB, wm, wn, lane, acc);
  }
  float* out = p.o0 + (int64_t)e * M * N;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + 32 * wm + 16 * i + 4 * (lane >> 4) + v;
        out[(int64_t)m * N + n0 + 32 * wn + 16 * j + (lane & 15)] = acc[i][j][v];
      }
}

inline bool dims_ok(int64_t R, int E, int a, int b) {
  return R >= 0 && E >= 1 && E <= kMaxE && a >= 64 && b >= 64 && a % 64 == 0 && b % 64 == 0;
}

template <int MODE>
int launch_rows(const Params& p, hipStream_t stream) {
  if (p.R == 0) return kOk;
  const int64_t gx = (p.R + BM - 1) / BM + p.E;  // >= sum over experts of ceil(count / 64)
  hipLaunchKernelGGL(rows_kernel<MODE>, dim3((unsigned)gx, (unsigned)(p.N / BN)), dim3(256), 0, stream, p);
  return launch_status();
}

}  // namespace f32g
}  // namespace moe

using namespace moe;
using namespace moe::f32g;

MOE_API int moe_grouped_gemm_f32_gate_up(const float* x, const float* w1, const float* w3, const int64_t* counts,
                                         int64_t n_rows, int32_t n_experts, int32_t dim, int32_t hidden, float* g,
                                         float* u, float* h, hipStream_t stream) {
  if (!dims_ok(n_rows, n_experts, dim, hidden)) return kErrInvalidArgument;
  if (n_rows > 0 && (!x || !w1 || !w3 || !counts || !g || !u || !h)) return kErrInvalidArgument;
  Params p{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.N = hidden; p.K = dim;
  p.a = x; p.b = w1; p.b2 = w3; p.o0 = g; p.o1 = u; p.o2 = h;
  return launch_rows<kGateUp>(p, stream);
}

MOE_API int moe_grouped_gemm_f32_down(const float* h, const float* w2, const int64_t* counts, int64_t n_rows,
                                      int32_t n_experts, int32_t dim, int32_t hidden, float* y, hipStream_t stream) {
  if (!dims_ok(n_rows, n_experts, dim, hidden)) return kErrInvalidArgument;
  if (n_rows > 0 && (!h || !w2 || !counts || !y)) return kErrInvalidArgument;
  Params p{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.N = dim; p.K = hidden;
  p.a = h; p.b = w2; p.o0 = y;
  return launch_rows<kDown>(p, stream);
}

MOE_API int moe_grouped_gemm_f32_bwd_dgu(const float* dy, const float* w2, const float* g, const float* u,
                                         const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                         int32_t hidden, float* dg, float* du, hipStream_t stream) {
  if (!dims_ok(n_rows, n_experts, dim, hidden)) return kErrInvalidArgument;
  if (n_rows > 0 && (!dy || !w2 || !g || !u || !counts || !dg || !du)) return kErrInvalidArgument;
  Params p{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.N = hidden; p.K = dim;
  p.a = dy; p.b = w2; p.g = g; p.u = u; p.o0 = dg; p.o1 = du;
  return launch_rows<kDgu>(p, stream);
}

MOE_API int moe_grouped_gemm_f32_bwd_dx(const float* dg, const float* du, const float* w1, const float* w3,
                                        const int64_t* counts, int64_t n_rows, int32_t n_experts, int32_t dim,
                                        int32_t hidden, float* dx, hipStream_t stream) {
  if (!dims_ok(n_rows, n_experts, dim, hidden)) return kErrInvalidArgument;
  if (n_rows > 0 && (!dg || !du || !w1 || !w3 || !counts || !dx)) return kErrInvalidArgument;
  Params p{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.N = dim; p.K = hidden;
  p.a = dg; p.a2 = du; p.b = w1; p.b2 = w3; p.o0 = dx;
  return launch_rows<kDx>(p, stream);
}

MOE_API int moe_grouped_gemm_f32_bwd_dw(const float* a, const float* b, const int64_t* counts, int64_t n_rows,
                                        int32_t n_experts, int32_t m, int32_t n, float* out, hipStream_t stream) {
  if (!dims_ok(n_rows, n_experts, m, n)) return kErrInvalidArgument;
  if (!counts || !out || (n_rows > 0 && (!a || !b))) return kErrInvalidArgument;
  Params p{};
  p.counts = counts; p.R = n_rows; p.E = n_experts; p.N = n; p.K = m;
  p.a = a; p.b = b; p.o0 = out;
  const int64_t tiles = (int64_t)(m / BM) * (n / BN);
  hipLaunchKernelGGL(dw_kernel, dim3((unsigned)n_experts, (unsigned)tiles), dim3(256), 0, stream, p);
  return launch_status();
}
