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

__global__ __launch_bounds__(256) void router_fwd_kernel(RouterFwdParams p) {
  __shared__ float s_choice[kRouterWaves][kRouterMaxE];
  __shared__ float s_score[kRouterWaves][kRouterMaxE];
  __shared__ uint32_t s_sel_e[kRouterWaves][kRouterMaxK];
  __shared__ uint32_t s_sel_key[kRouterWaves][kRouterMaxK];
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

  for (int64_t t = (int64_t)blockIdx.x * kRouterWaves + wv; t < p.n_tokens;
       t += (int64_t)gridDim.x * kRouterWaves) {
    const float* lrow = p.logits + t * E;
    float s[kRouterMaxQ];
#pragma unroll
    for (int q = 0; q < kRouterMaxQ; ++q) {
      const int e = lane + kWave * q;
      s[q] = (q < nq && e < E) ? lrow[e] : -INFINITY;
    }

    if (p.score_func == kSigmoid) {
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) s[q] = 1.0f / (1.0f + expf(-s[q]));
    } else {
      float m = s[0];
#pragma unroll
      for (int q = 1; q < kRouterMaxQ; ++q)
        if (q < sm_iters) m = (m > s[q]) ? m : s[q];
      for (int off = sm_width >> 1; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off);
        m = (m < o) ? o : m;
      }
      float sum = 0.0f;
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q)
        if (q < sm_iters) {
          s[q] = expf(s[q] - m);
          sum += s[q];
        }
      for (int off = sm_width >> 1; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) s[q] = s[q] / sum;
    }

    float c[kRouterMaxQ];
#pragma unroll
    for (int q = 0; q < kRouterMaxQ; ++q) {
      const int e = lane + kWave * q;
      if (q < nq && e < E) {
        p.scores[t * E + e] = s[q];
        s_score[wv][e] = s[q];
        c[q] = p.bias ? s[q] + p.bias[e] : s[q];
      } else {
        c[q] = -INFINITY;
      }
    }

    if (p.n_groups > 0) {
      // group score = sum of the two largest choice scores of the group
      const int epg = E / p.n_groups;
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) {
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
      for (int q = 0; q < kRouterMaxQ; ++q) {
        const int e = lane + kWave * q;
        if (q < nq && e < E && !((gmask >> (e / epg)) & 1ull)) c[q] = -INFINITY;
      }
    }

    if (!p.force_lb) {
      // Top-k by (radix key desc, expert index asc): the set torch's radix
      // select keeps, including its lowest-index-first rule among ties.
      uint32_t keyq[kRouterMaxQ];
#pragma unroll
      for (int q = 0; q < kRouterMaxQ; ++q) keyq[q] = radix_key(c[q]);
      uint32_t taken = 0;
      for (int j = 0; j < K; ++j) {
        uint64_t best = 0;
#pragma unroll
        for (int q = 0; q < kRouterMaxQ; ++q) {
          const int e = lane + kWave * q;
          if (q < nq && e < E && !((taken >> q) & 1u)) {
            const uint64_t v = ((uint64_t)keyq[q] << 32) | (uint32_t)(~e);
            best = v > best ? v : best;
          }
        }
        best = wave_max_u64(best);
        const uint32_t es = ~(uint32_t)best;
        if ((int)(es & 63u) == lane) taken |= 1u << (es >> 6);
        if (lane == 0) {
          s_sel_e[wv][j] = es;
          s_sel_key[wv][j] = (uint32_t)(best >> 32);
        }
      }
    } else if (lane < K) {
      s_sel_e[wv][lane] = (uint32_t)((t * K + lane) % E);
    }
    wave_lds_sync();

    // Output slot order of torch.topk(sorted=False) on the GPU: first every
    // selected expert whose key is strictly above the k-th key, by ascending
    // index, then the k-th-key ties, by ascending index.
    float ts0 = 0.0f;
    int slot = lane;
    uint32_t my_e = 0;
    if (lane < K) {
      my_e = s_sel_e[wv][lane];
      ts0 = s_score[wv][my_e];
      if (!p.force_lb) {
        const uint32_t kth = s_sel_key[wv][K - 1];
        const int my_cls = s_sel_key[wv][lane] > kth ? 0 : 1;
        slot = 0;
        for (int i = 0; i < K; ++i) {
          const int ci = s_sel_key[wv][i] > kth ? 0 : 1;
          const uint32_t ei = s_sel_e[wv][i];
          slot += (ci < my_cls) || (ci == my_cls && ei < my_e);
        }
      }
    }
    wave_lds_sync();
    if (lane < K) {
      s_ts[wv][slot] = ts0;
      p.indices[t * K + slot] = (int64_t)my_e;
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
  hipLaunchKernelGGL(router_fwd_kernel, dim3(router_grid(n_tokens)), dim3(256), 0, stream, p);
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
