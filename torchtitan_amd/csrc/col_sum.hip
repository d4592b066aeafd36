// Per-expert column sums of routed rows on MI355X: the bias gradients of the
// gpt-oss experts.
//
// The reference adds the expert biases to the grouped-GEMM outputs through
// bias.repeat_interleave(num_tokens_per_expert) (torchtitan/models/gpt_oss/
// moe.py:104-121), whose backward sums each expert's gradient rows into its
// bias row (an index_add over the routed rows). Here
//   out[e * ld_out + c * col_stride] = sum over the rows r of expert e of src[r * ld_src + c]
// in fp32, in a fixed order (bit-reproducible), for bf16 src.
//
// Block per (expert, 64 columns): 256 threads = 8 column chunks of 8 x 32 row
// lanes; each thread accumulates its chunk over every 32nd row (four 16-byte
// loads in flight), then the 32 row lanes are added in LDS in lane order.
#include "common.h"

namespace moe {

__global__ __launch_bounds__(256) void grouped_col_sum_kernel(const uint16_t* __restrict__ src, int64_t ld_src,
                                                              const int64_t* __restrict__ counts, int64_t R, int E,
                                                              int C, float* __restrict__ out, int64_t ld_out,
                                                              int col_stride) {
  __shared__ float s_red[32][65];
  __shared__ int s_tmp[8];
  __shared__ int s_seg[2];
  const int nc = C / 64;
  const int e = blockIdx.x / nc;
  const int c0 = (blockIdx.x % nc) * 64;
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
    for (int i = 0; i < 4; ++i)
      if (threadIdx.x * 4 + i == e) { s_seg[0] = st[i]; s_seg[1] = cnt[i]; }
    __syncthreads();
  }
  const int64_t seg0 = s_seg[0];
  int64_t n = s_seg[1];
  if (seg0 + n > R) n = R - seg0 > 0 ? R - seg0 : 0;
  const int ch = threadIdx.x & 7, rl = threadIdx.x >> 3;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  const uint16_t* base = src + seg0 * ld_src + c0 + ch * 8;
  for (int64_t r = rl; r < n; r += 128) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      v[u] = (r + 32 * u < n) ? *(const uint4*)(base + (r + 32 * u) * ld_src) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[0] += bf_lo(v[u].x); acc[1] += bf_hi(v[u].x);
      acc[2] += bf_lo(v[u].y); acc[3] += bf_hi(v[u].y);
      acc[4] += bf_lo(v[u].z); acc[5] += bf_hi(v[u].z);
      acc[6] += bf_lo(v[u].w); acc[7] += bf_hi(v[u].w);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) s_red[rl][ch * 8 + j] = acc[j];
  __syncthreads();
  if (threadIdx.x < 64) {
    float s = 0.f;
    for (int i = 0; i < 32; ++i) s += s_red[i][threadIdx.x];
    out[(int64_t)e * ld_out + (int64_t)(c0 + threadIdx.x) * col_stride] = s;
  }
}

}  // namespace moe

using namespace moe;

MOE_API int moe_grouped_col_sum(const uint16_t* src, int64_t ld_src, const int64_t* counts, int64_t n_rows,
                                int32_t n_experts, int32_t cols, float* out, int64_t ld_out, int32_t col_stride,
                                hipStream_t stream) {
  if (n_rows < 0 || n_experts < 1 || n_experts > 1024 || cols < 64 || cols % 64 || col_stride < 1)
    return kErrInvalidArgument;
  if (ld_src < cols || ld_src % 8 || ld_out < (int64_t)(cols - 1) * col_stride + 1) return kErrInvalidArgument;
  if (!counts || !out || (n_rows > 0 && !src)) return kErrInvalidArgument;
  hipLaunchKernelGGL(grouped_col_sum_kernel, dim3(n_experts * (cols / 64)), dim3(256), 0, stream, src, ld_src, counts,
                     n_rows, n_experts, cols, out, ld_out, col_stride);
  return launch_status();
}
