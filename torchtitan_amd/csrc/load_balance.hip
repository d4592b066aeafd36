// Auxiliary-loss-free expert-bias update on MI355X: one launch for every MoE
// layer of a model.
//
// Replaces _update_expert_bias in register_moe_load_balancing_hook,
// torchtitan/components/optimizer.py:366-437, run as an optimizer step
// pre-hook. Per layer, with t = tokens_per_expert (fp32, integer-valued):
//   t     <- floor(t / 2)                 if the block recomputes (AC), :389-394
//   delta  = coeff * sign(mean(t) - t)                                  :424-426
//   delta  = delta - mean(delta)                                        :427
//   expert_bias += delta ; tokens_per_expert <- 0                       :429-431
// One workgroup per layer. The cross-rank all-reduce of the counts (:400-414)
// is the caller's (one GPU here). mean(t) is exact while sum(t) < 2^24 (the
// counts are integers); mean(delta) sums multiples of coeff and may differ from
// torch's reduction order in the last bits.
#include "common.h"

namespace moe {

constexpr int kMaxBalanceLayers = 64;
constexpr int kMaxBalanceExperts = 1024;

struct BalanceParams {
  float* tokens_per_expert[kMaxBalanceLayers];
  float* expert_bias[kMaxBalanceLayers];
  float coeff[kMaxBalanceLayers];
  int halve[kMaxBalanceLayers];
  int E;
};

__device__ __forceinline__ float block_sum256(float v, float* tmp) {
  v = wave_sum_f32(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) tmp[wv] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) s += tmp[w];
  __syncthreads();
  return s;
}

__device__ __forceinline__ float sign_f(float x) {
  return x > 0.f ? 1.f : (x < 0.f ? -1.f : (x == 0.f ? 0.f : x));  // NaN stays NaN, as torch.sign
}

__global__ __launch_bounds__(256) void bias_update_kernel(BalanceParams p) {
  __shared__ float tmp[4];
  const int l = blockIdx.x;
  float* tpe = p.tokens_per_expert[l];
  float* bias = p.expert_bias[l];
  const int E = p.E;
  float t[4];
  float local = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = threadIdx.x + i * 256;
    float v = (e < E) ? tpe[e] : 0.f;
    if (p.halve[l]) v = floorf(v / 2.0f);
    t[i] = v;
    local += v;
  }
  const float mean_t = block_sum256(local, tmp) / (float)E;
  float d[4];
  float dl = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = threadIdx.x + i * 256;
    d[i] = (e < E) ? p.coeff[l] * sign_f(mean_t - t[i]) : 0.f;
    dl += d[i];
  }
  const float mean_d = block_sum256(dl, tmp) / (float)E;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = threadIdx.x + i * 256;
    if (e < E) {
      bias[e] = bias[e] + (d[i] - mean_d);
      tpe[e] = 0.f;
    }
  }
}

}  // namespace moe

using namespace moe;

MOE_API int moe_expert_bias_update(float* const* tokens_per_expert, float* const* expert_bias,
                                   const float* coeff, const int32_t* halve, int32_t n_layers,
                                   int32_t n_experts, hipStream_t stream) {
  if (n_layers < 0 || n_layers > kMaxBalanceLayers || n_experts < 1 || n_experts > kMaxBalanceExperts)
    return kErrInvalidArgument;
  if (n_layers == 0) return kOk;
  if (!tokens_per_expert || !expert_bias || !coeff || !halve) return kErrInvalidArgument;
  BalanceParams p{};
  for (int l = 0; l < n_layers; ++l) {
    if (!tokens_per_expert[l] || !expert_bias[l]) return kErrInvalidArgument;
    p.tokens_per_expert[l] = tokens_per_expert[l];
    p.expert_bias[l] = expert_bias[l];
    p.coeff[l] = coeff[l];
    p.halve[l] = halve[l] ? 1 : 0;
  }
  p.E = n_experts;
  hipLaunchKernelGGL(bias_update_kernel, dim3(n_layers), dim3(256), 0, stream, p);
  return launch_status();
}
