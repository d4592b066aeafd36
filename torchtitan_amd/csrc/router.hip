// Token-choice top-k router for MI355X.
//
// One 64-wide wavefront routes one token: lane l owns experts l, l+64, ...
// (the same lane/expert layout torch's persistent warp softmax uses on a
// 64-wide wave), so scores, the group-limited mask, top-k selection, the
// gather of un-biased scores, route_norm and route_scale all stay in
// registers and per-wave LDS. The logits come from the caller: by default
// torch's fp32 gate GEMM under autocast, the reference's own call.
//
// Follows torchtitan/models/common/moe.py:
//   score function            :236-241
//   + expert_bias (selection) :243
//   group-limited mask        :169-209
//   top-k (sorted=False)      :247-249
//   gather un-biased scores   :254
//   debug round-robin         :152-167, :257-261
//   route_norm / route_scale  :263-266
#include "common.h"

namespace moe {

constexpr int kRouterMaxE = 512;
constexpr int kRouterMaxQ = kRouterMaxE / kWave;  // experts per lane
constexpr int kRouterMaxK = 64;
constexpr int kRouterWaves = 4;

enum ScoreFunc : int { kSoftmax = 0, kSigmoid = 1 };

// v from another lane of the same 16-lane row (DPP control CTRL; all lanes active)
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_from(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
// Wave-uniform maximum / minimum of a 32-bit value: four DPP exchanges (lane xor 1,
// xor 2, the half-row mirror, the row mirror) leave every lane of a 16-lane row
// holding the row's extreme; the four rows are then read from lanes 0, 16, 32, 48.
// No LDS round trips, unlike shuffles through ds_bpermute.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_extreme_u32(uint32_t v) {
  auto pick = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  v = pick(v, dpp_from<0xb1>(v));   // quad_perm [1, 0, 3, 2]
  v = pick(v, dpp_from<0x4e>(v));   // quad_perm [2, 3, 0, 1]
  v = pick(v, dpp_from<0x141>(v));  // row_half_mirror
  v = pick(v, dpp_from<0x140>(v));  // row_mirror
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return pick(pick(r0, r1), pick(r2, r3));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return wave_extreme_u32<true>(v); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return wave_extreme_u32<false>(v); }

struct RouterFwdParams {
  const float* logits;
  const float* bias;  // nullable
  int64_t n_tokens;
  int n_experts, top_k, score_func, n_groups, n_limited, route_norm, force_lb;
  float route_scale;
  float* scores;      // [N, E]
  float* top_scores;  // [N, K]
  int64_t* indices;   // [N, K]
};

// NQ experts per lane: max(1, next power of two of E / 64), which is also the
// number of elements each lane visits in torch's warp softmax for that E.
template <int NQ>
__global__ __launch_bounds__(256) void router_fwd_kernel(RouterFwdParams p) {
  __shared__ float s_choice[kRouterWaves][kRouterMaxE];
  __shared__ float s_score[kRouterWaves][kRouterMaxE];
  __shared__ float s_ts[kRouterWaves][kRouterMaxK];

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int E = p.n_experts, K = p.top_k;
  const int nq = (E + 63) >> 6;
  // torch's warp softmax: next power of two of E spread over min(pow2, 64)
  // lanes, each lane visiting pow2/width elements strided by the width.
  int pow2 = 1;
  while (pow2 < E) pow2 <<= 1;
  const int sm_width = pow2 < kWave ? pow2 : kWave;
  const int sm_iters = pow2 / sm_width;
  // the lane's expert biases, loaded once: read inside the token loop they would wait
  // behind that token's score stores (loads and stores share one counter)
  float bq[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int e = lane + kWave * q;
    bq[q] = (p.bias && q < nq && e < E) ? p.bias[e] : 0.0f;
  }

  for (int64_t t = (int64_t)blockIdx.x * kRouterWaves + wv; t < p.n_tokens;
       t += (int64_t)gridDim.x * kRouterWaves) {
    const float* lrow = p.logits + t * E;
    float s[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int e = lane + kWave * q;
      s[q] = (q < nq && e < E) ? lrow[e] : -INFINITY;
    }

    if (p.score_func == kSigmoid) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) s[q] = 1.0f / (1.0f + expf(-s[q]));
    } else {
      float m = s[0];
#pragma unroll
      for (int q = 1; q < NQ; ++q)
        if (q < sm_iters) m = (m > s[q]) ? m : s[q];
      for (int off = sm_width >> 1; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off);
        m = (m < o) ? o : m;
      }
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        if (q < sm_iters) {
          s[q] = expf(s[q] - m);
          sum += s[q];
        }
      for (int off = sm_width >> 1; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
#pragma unroll
      for (int q = 0; q < NQ; ++q) s[q] = s[q] / sum;
    }

    float c[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int e = lane + kWave * q;
      if (q < nq && e < E) {
        p.scores[t * E + e] = s[q];
        s_score[wv][e] = s[q];
        c[q] = p.bias ? s[q] + bq[q] : s[q];
      } else {
        c[q] = -INFINITY;
      }
    }

    if (p.n_groups > 0) {
      // group score = sum of the two largest choice scores of the group
      const int epg = E / p.n_groups;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int e = lane + kWave * q;
        if (q < nq && e < E) s_choice[wv][e] = c[q];
      }
      wave_lds_sync();
      uint32_t gkey = 0;
      if (lane < p.n_groups) {
        uint32_t k1 = 0, k2 = 0;
        float v1 = 0.0f, v2 = 0.0f;
        for (int i = 0; i < epg; ++i) {
          const float x = s_choice[wv][lane * epg + i];
          const uint32_t k = radix_key(x);
          if (k > k1) {
            k2 = k1; v2 = v1; k1 = k; v1 = x;
          } else if (k > k2) {
            k2 = k; v2 = x;
          }
        }
        gkey = radix_key(v1 + v2);
      }
      uint64_t gmask = 0;
      bool gtaken = false;
      for (int j = 0; j < p.n_limited; ++j) {
        uint64_t v = (lane < p.n_groups && !gtaken) ? (((uint64_t)gkey << 32) | (uint32_t)(~lane)) : 0ull;
        v = wave_max_u64(v);
        const int g = (int)(~(uint32_t)v);
        gmask |= 1ull << g;
        if (lane == g) gtaken = true;
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int e = lane + kWave * q;
        if (q < nq && e < E && !((gmask >> (e / epg)) & 1ull)) c[q] = -INFINITY;
      }
    }

    float ts0 = 0.0f;
    int slot = lane;
    uint32_t my_e = 0;
    if (!p.force_lb) {
      // Top-k by (radix key desc, expert index asc): the set torch's radix select
      // keeps, including its lowest-index-first rule among ties. Each round takes
      // every lane's best remaining key (the lowest q among equal keys: e = lane + 64 q),
      // the wave maximum of those, and the winning lane from a ballot; only when
      // several lanes hold that key does a second reduction pick the lowest expert.
      // Keys are never 0 (radix_key), so 0 marks "no candidate".
      uint32_t keyo[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int e = lane + kWave * q;
        keyo[q] = (q < nq && e < E) ? radix_key(c[q]) : 0u;
      }
      uint32_t taken = 0, kth = 0;
      for (int j = 0; j < K; ++j) {
        uint32_t lk = 0;
        int lq = 0;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const uint32_t k = ((taken >> q) & 1u) ? 0u : keyo[q];
          if (k > lk) { lk = k; lq = q; }
        }
        const uint32_t best = wave_max_u32(lk);
        const bool mine = lk == best && lk != 0;
        const uint64_t m = __ballot(mine);
        uint32_t win_e;
        if (__popcll(m) == 1) {
          const int wl = __builtin_ctzll(m);
          win_e = (uint32_t)(wl + kWave * __builtin_amdgcn_readlane(lq, wl));
        } else {
          win_e = wave_min_u32(mine ? (uint32_t)(lane + kWave * lq) : 0xffffffffu);
        }
        if ((int)(win_e & 63u) == lane) taken |= 1u << (win_e >> 6);
        kth = best;
      }
      // Output slot order of torch.topk(sorted=False) on the GPU: first every selected
      // expert whose key is strictly above the k-th key, by ascending index, then the
      // k-th-key ties, by ascending index. Column q holds experts 64 q .. 64 q + 63, so
      // an expert's rank in its class is the class members of the earlier columns plus
      // those of lower lanes in its own column.
      uint64_t above[NQ], ties[NQ];
      int n_above = 0;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const bool sel = (taken >> q) & 1u;
        above[q] = __ballot(sel && keyo[q] > kth);
        ties[q] = __ballot(sel && keyo[q] == kth);
        n_above += __popcll(above[q]);
      }
      int before_a = 0, before_t = n_above;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        if ((taken >> q) & 1u) {
          const bool a = keyo[q] > kth;
          const uint64_t mq = a ? above[q] : ties[q];
          const int r = (a ? before_a : before_t) +
                        (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mq >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mq, 0u));
          s_ts[wv][r] = s[q];
          p.indices[t * K + r] = (int64_t)(lane + kWave * q);
        }
        before_a += __popcll(above[q]);
        before_t += __popcll(ties[q]);
      }
    } else {
      wave_lds_sync();  // s_score of every lane
      if (lane < K) {
        my_e = (uint32_t)((t * K + lane) % E);
        ts0 = s_score[wv][my_e];
      }
      wave_lds_sync();
      if (lane < K) {
        s_ts[wv][slot] = ts0;
        p.indices[t * K + slot] = (int64_t)my_e;
      }
    }
    wave_lds_sync();
    float v = (lane < K) ? s_ts[wv][lane] : 0.0f;
    if (p.route_norm) {
      const float den = wave_torch_row_sum(v, K) + 1e-20f;
      v = v / den;
    }
    v = v * p.route_scale;
    if (lane < K) p.top_scores[t * K + lane] = v;
    wave_lds_sync();
  }
}

struct RouterBwdParams {
  const float* grad_top_scores;  // [N, K]
  const float* scores;           // [N, E] saved score-function output
  const int64_t* indices;        // [N, K]
  int64_t n_tokens;
  int n_experts, top_k, score_func, route_norm;
  float route_scale;
  float* grad_logits;  // [N, E]
};

// Backward of moe.py:236-266 (autograd of scale, norm, gather, sigmoid or
// softmax), producing d(logits) for torch's gate GEMM backward.
__global__ __launch_bounds__(256) void router_bwd_kernel(RouterBwdParams p) {
  __shared__ float s_g[kRouterWaves][kRouterMaxE];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int E = p.n_experts, K = p.top_k;
  const int nq = (E + 63) >> 6;
  int pow2 = 1;
  while (pow2 < E) pow2 <<= 1;
  const int sm_width = pow2 < kWave ? pow2 : kWave;

  for (int64_t t = (int64_t)blockIdx.x * kRouterWaves + wv; t < p.n_tokens;
       t += (int64_t)gridDim.x * kRouterWaves) {
    float g = 0.0f, s0 = 0.0f;
    int e = 0;
    if (lane < K) {
      g = p.grad_top_scores[t * K + lane];
      e = (int)p.indices[t * K + lane];
      s0 = p.scores[t * E + e];
    }
    const float g1 = g * p.route_scale;
    float gts0 = g1;
    if (p.route_norm) {
      const float den = wave_torch_row_sum(s0, K) + 1e-20f;
      const float ga = g1 / den;
      const float gd = -g1 * ((s0 / den) / den);
      const float gden = wave_torch_row_sum(gd, K);
      gts0 = ga + gden;
    }
#pragma unroll
    for (int q = 0; q < kRouterMaxQ; ++q) {
      const int ee = lane + kWave * q;
      if (q < nq && ee < E) s_g[wv][ee] = 0.0f;
    }
    wave_lds_sync();
    if (lane < K) s_g[wv][e] = 0.0f + gts0;
    wave_lds_sync();
    const float* srow = p.scores + t * E;
    float* grow = p.grad_logits + t * E;
    if (p.score_func == kSigmoid) {
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) {
        const int ee = lane + kWave * q;
        if (q < nq && ee < E) {
          const float sc = srow[ee];
          grow[ee] = (s_g[wv][ee] * (1.0f - sc)) * sc;
        }
      }
    } else {
      float dot = 0.0f;
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) {
        const int ee = lane + kWave * q;
        if (q < nq && ee < E) dot += s_g[wv][ee] * srow[ee];
      }
      for (int off = sm_width >> 1; off > 0; off >>= 1) dot += __shfl_xor(dot, off);
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) {
        const int ee = lane + kWave * q;
        if (q < nq && ee < E) {
          const float sc = srow[ee];
          grow[ee] = sc * (s_g[wv][ee] - dot);
        }
      }
    }
    wave_lds_sync();
  }
}

static int router_grid(int64_t n_tokens) {
  int64_t g = (n_tokens + kRouterWaves - 1) / kRouterWaves;
  if (g > 16384) g = 16384;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace moe

using namespace moe;

MOE_API int moe_router_fwd(const float* logits, const float* expert_bias, int64_t n_tokens,
                           int32_t n_experts, int32_t top_k, int32_t score_func,
                           int32_t n_expert_groups, int32_t n_limited_groups, int32_t route_norm,
                           float route_scale, int32_t force_load_balance, float* scores,
                           float* top_scores, int64_t* selected_experts, hipStream_t stream) {
  if (n_tokens < 0 || n_experts < 1 || n_experts > kRouterMaxE || top_k < 1 || top_k > kRouterMaxK ||
      top_k > n_experts || (score_func != kSoftmax && score_func != kSigmoid))
    return kErrInvalidArgument;
  if (n_expert_groups > 0) {
    if (n_expert_groups > kWave || n_experts % n_expert_groups != 0 ||
        n_experts / n_expert_groups < 2 || n_limited_groups < 1 || n_limited_groups > n_expert_groups)
      return kErrInvalidArgument;
  }
  if (n_tokens == 0) return kOk;
  if (!logits || !scores || !top_scores || !selected_experts) return kErrInvalidArgument;
  RouterFwdParams p{logits, expert_bias, n_tokens, n_experts, top_k, score_func,
                    n_expert_groups > 0 ? n_expert_groups : 0, n_limited_groups, route_norm,
                    force_load_balance, route_scale, scores, top_scores, selected_experts};
  const dim3 grid(router_grid(n_tokens));
  if (n_experts <= 64) hipLaunchKernelGGL(router_fwd_kernel<1>, grid, dim3(256), 0, stream, p);
  else if (n_experts <= 128) hipLaunchKernelGGL(router_fwd_kernel<2>, grid, dim3(256), 0, stream, p);
  else if (n_experts <= 256) hipLaunchKernelGGL(router_fwd_kernel<4>, grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL(router_fwd_kernel<kRouterMaxQ>, grid, dim3(256), 0, stream, p);
  return launch_status();
}

MOE_API int moe_router_bwd(const float* grad_top_scores, const float* scores,
                           const int64_t* selected_experts, int64_t n_tokens, int32_t n_experts,
                           int32_t top_k, int32_t score_func, int32_t route_norm, float route_scale,
                           float* grad_logits, hipStream_t stream) {
  if (n_tokens < 0 || n_experts < 1 || n_experts > kRouterMaxE || top_k < 1 || top_k > kRouterMaxK ||
      top_k > n_experts || (score_func != kSoftmax && score_func != kSigmoid))
    return kErrInvalidArgument;
  if (n_tokens == 0) return kOk;
  if (!grad_top_scores || !scores || !selected_experts || !grad_logits) return kErrInvalidArgument;
  RouterBwdParams p{grad_top_scores, scores, selected_experts, n_tokens, n_experts, top_k,
                    score_func, route_norm, route_scale, grad_logits};
  hipLaunchKernelGGL(router_bwd_kernel, dim3(router_grid(n_tokens)), dim3(256), 0, stream, p);
  return launch_status();
}
