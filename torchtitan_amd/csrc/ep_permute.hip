// Expert-parallel local permute on MI355X: rank-major -> expert-major gather
// indices and the row movement that uses them.
//
// Replaces _generate_permute_indices, _permute and _unpermute of
// torchtitan/distributed/expert_parallel.py:26-80. After the token all-to-all
// of expert parallelism a rank holds, for each source rank r and local expert
// e, a segment of counts[r * E + e] rows, in rank-major order; the grouped
// GEMMs need them expert-major. Segment s = e * R + r (expert-major) starts at
// in_start = exclusive cumsum of counts in rank-major order and lands at
// out_start = exclusive cumsum of the expert-major lengths; output position p of
// segment s reads input row in_start[s] + (p - out_start[s]).
//
// One kernel computes both scans in LDS per workgroup (R * E <= 2048 segments)
// and fills the positions grid-stride; the reference's host sync on the total
// (torch.arange(total)) becomes the caller's `total` argument. Positions past
// the sum of the counts (a `total` larger than it) are set to -1.
#include "common.h"

namespace moe {

constexpr int kMaxEpSegments = 2048;

// inclusive scan of v over the 256 threads of the block (v: each thread's total)
__device__ __forceinline__ int64_t block_inclusive_scan_i64(int64_t v, int64_t* tmp) {
  tmp[threadIdx.x] = v;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int64_t o = threadIdx.x >= off ? tmp[threadIdx.x - off] : 0;
    __syncthreads();
    tmp[threadIdx.x] += o;
    __syncthreads();
  }
  const int64_t r = tmp[threadIdx.x];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(256) void ep_permute_indices_kernel(const int64_t* __restrict__ counts, int R, int E,
                                                                 int64_t total, int64_t* __restrict__ out_idx,
                                                                 int64_t* __restrict__ tokens_per_expert) {
  __shared__ int64_t s_in[kMaxEpSegments];    // input start of expert-major segment s
  __shared__ int64_t s_out[kMaxEpSegments + 1];
  __shared__ int64_t tmp[256];
  const int n = R * E;
  constexpr int PER = kMaxEpSegments / 256;
  // rank-major exclusive scan -> input starts
  {
    int64_t v[PER];
    int64_t run = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = threadIdx.x * PER + i;
      v[i] = f < n ? counts[f] : 0;
      run += v[i];
    }
    int64_t base = block_inclusive_scan_i64(run, tmp) - run;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = threadIdx.x * PER + i;
      if (f < n) {
        const int r = f / E, e = f - r * E;
        s_in[e * R + r] = base;  // rank-major position f -> expert-major segment e R + r
      }
      base += v[i];
    }
  }
  // expert-major exclusive scan of the lengths -> output starts
  {
    int64_t v[PER];
    int64_t run = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int s = threadIdx.x * PER + i;
      int64_t len = 0;
      if (s < n) {
        const int e = s / R, r = s - e * R;
        len = counts[r * E + e];
      }
      v[i] = len;
      run += len;
    }
    const int64_t incl = block_inclusive_scan_i64(run, tmp);
    int64_t base = incl - run;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int s = threadIdx.x * PER + i;
      if (s < n) s_out[s] = base;
      base += v[i];
    }
    if (threadIdx.x == 255) s_out[n] = incl;  // the sum of every count
    __syncthreads();
  }
  if (blockIdx.x == 0 && tokens_per_expert) {
    for (int e = threadIdx.x; e < E; e += 256) {
      int64_t s = 0;
      for (int r = 0; r < R; ++r) s += counts[r * E + e];
      tokens_per_expert[e] = s;
    }
  }
  const int64_t sum = s_out[n];
  for (int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x; p < total; p += (int64_t)gridDim.x * 256) {
    if (p >= sum) {
      out_idx[p] = -1;
      continue;
    }
    int lo = 0, hi = n - 1;  // last segment with s_out <= p (empty segments share starts)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_out[mid] <= p) lo = mid; else hi = mid - 1;
    }
    out_idx[p] = s_in[lo] + (p - s_out[lo]);
  }
}

// dst[i] = src[idx[i]] (gather) or dst[idx[i]] = src[i] (scatter), rows of D
// elements moved as 16-byte chunks.
template <bool SCATTER>
__global__ __launch_bounds__(256) void move_rows_kernel(const uint4* __restrict__ src, const int64_t* __restrict__ idx,
                                                        int64_t n_rows, int64_t n_src_rows, int cpr,
                                                        uint4* __restrict__ dst) {
  const int64_t total = n_rows * cpr;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total; c += (int64_t)gridDim.x * 256) {
    const int64_t i = c / cpr;
    const int ch = (int)(c - i * cpr);
    const int64_t j = idx[i];
    if (j < 0 || j >= n_src_rows) continue;  // -1 marks positions past the counts
    if (SCATTER) dst[j * cpr + ch] = src[i * cpr + ch];
    else dst[i * cpr + ch] = src[j * cpr + ch];
  }
}

}  // namespace moe

using namespace moe;

MOE_API int moe_ep_permute_indices(const int64_t* tokens_per_expert_group, int32_t experts_per_rank,
                                   int32_t num_ranks, int64_t total, int64_t* permuted_indices,
                                   int64_t* num_tokens_per_expert, hipStream_t stream) {
  if (experts_per_rank < 1 || num_ranks < 1 || total < 0) return kErrInvalidArgument;
  if ((int64_t)experts_per_rank * num_ranks > kMaxEpSegments) return kErrUnsupportedShape;
  if (!tokens_per_expert_group || (total > 0 && !permuted_indices)) return kErrInvalidArgument;
  int64_t g = (total + 255) / 256;
  if (g > 1024) g = 1024;
  if (g < 1) g = 1;
  hipLaunchKernelGGL(ep_permute_indices_kernel, dim3((int)g), dim3(256), 0, stream, tokens_per_expert_group,
                     num_ranks, experts_per_rank, total, permuted_indices, num_tokens_per_expert);
  return launch_status();
}

static int move_rows(const void* src, const int64_t* idx, int64_t n_rows, int64_t n_other_rows, int32_t dim,
                     int32_t dtype, void* dst, bool scatter, hipStream_t stream) {
  if (n_rows < 0 || n_other_rows < 0 || dim < 1) return kErrInvalidArgument;
  const int esize = dtype == MOE_DTYPE_BF16 ? 2 : (dtype == MOE_DTYPE_FP32 ? 4 : 0);
  if (!esize || ((int64_t)dim * esize) % 16) return kErrUnsupportedShape;
  if (n_rows == 0) return kOk;
  if (!src || !idx || !dst) return kErrInvalidArgument;
  const int cpr = (int)((int64_t)dim * esize / 16);
  int64_t g = (n_rows * cpr + 255) / 256;
  if (g > 16384) g = 16384;
  if (scatter)
    hipLaunchKernelGGL(move_rows_kernel<true>, dim3((int)g), dim3(256), 0, stream, (const uint4*)src, idx, n_rows,
                       n_other_rows, cpr, (uint4*)dst);
  else
    hipLaunchKernelGGL(move_rows_kernel<false>, dim3((int)g), dim3(256), 0, stream, (const uint4*)src, idx, n_rows,
                       n_other_rows, cpr, (uint4*)dst);
  return launch_status();
}

MOE_API int moe_gather_rows(const void* src, int64_t n_src_rows, const int64_t* idx, int64_t n_rows, int32_t dim,
                            int32_t dtype, void* dst, hipStream_t stream) {
  return move_rows(src, idx, n_rows, n_src_rows, dim, dtype, dst, false, stream);
}

MOE_API int moe_scatter_rows(const void* src, const int64_t* idx, int64_t n_rows, int32_t dim, int32_t dtype,
                             void* dst, int64_t n_dst_rows, hipStream_t stream) {
  return move_rows(src, idx, n_rows, n_dst_rows, dim, dtype, dst, true, stream);
}
