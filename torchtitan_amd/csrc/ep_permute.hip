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
// With a pad multiple (torchao's permute_and_pad, called at
// expert_parallel.py:537-551 for the fp8 / MXFP8 grouped GEMMs), every
// expert's group is followed by zero rows up to a multiple of it.
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

// pad > 1 (permute_and_pad): every expert's group is padded with zero rows to a
// multiple of pad; padding positions read the zero row appended after the
// n_in input rows (index n_in), tokens_per_expert gets the padded counts and
// group_offsets (nullable) the inclusive int32 ends of the padded groups.
__global__ __launch_bounds__(256) void ep_permute_indices_kernel(const int64_t* __restrict__ counts, int R, int E,
                                                                 int pad, int64_t total, int64_t* __restrict__ out_idx,
                                                                 int64_t* __restrict__ tokens_per_expert,
                                                                 int32_t* __restrict__ group_offsets) {
  __shared__ int64_t s_in[kMaxEpSegments];    // input start of expert-major segment s
  __shared__ int64_t s_out[kMaxEpSegments + 1];
  __shared__ int64_t s_len[kMaxEpSegments];
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
  // expert-major exclusive scan of the lengths (each expert's last segment
  // carrying its group's padding) -> output starts
  int64_t n_in = 0;
  {
    int64_t v[PER];
    int64_t run = 0, run_in = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int s = threadIdx.x * PER + i;
      int64_t len = 0, padded = 0;
      if (s < n) {
        const int e = s / R, r = s - e * R;
        len = counts[r * E + e];
        padded = len;
        if (pad > 1 && r == R - 1) {  // the group's padding follows its last segment
          int64_t g = 0;
          for (int rr = 0; rr < R; ++rr) g += counts[rr * E + e];
          padded += (g + pad - 1) / pad * pad - g;
        }
        s_len[s] = len;
      }
      v[i] = padded;
      run += padded;
      run_in += len;
    }
    const int64_t incl = block_inclusive_scan_i64(run, tmp);
    n_in = block_inclusive_scan_i64(run_in, tmp);
    if (threadIdx.x == 255) tmp[0] = n_in;
    int64_t base = incl - run;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int s = threadIdx.x * PER + i;
      if (s < n) s_out[s] = base;
      base += v[i];
    }
    if (threadIdx.x == 255) s_out[n] = incl;  // the padded total
    __syncthreads();
    n_in = tmp[0];  // the sum of every count (the zero row's index)
    __syncthreads();
  }
  if (blockIdx.x == 0 && (tokens_per_expert || group_offsets)) {
    for (int e = threadIdx.x; e < E; e += 256) {
      int64_t g = 0;
      for (int r = 0; r < R; ++r) g += counts[r * E + e];
      if (pad > 1) g = (g + pad - 1) / pad * pad;
      if (tokens_per_expert) tokens_per_expert[e] = g;
      if (group_offsets) group_offsets[e] = (int32_t)(s_out[e * R] + g);  // the group's segments are contiguous
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
    const int64_t off = p - s_out[lo];
    out_idx[p] = off < s_len[lo] ? s_in[lo] + off : n_in;  // past the rows: the group's padding
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
    if (SCATTER) {
      if (j >= 0 && j < n_src_rows) dst[j * cpr + ch] = src[i * cpr + ch];
    } else if (j == n_src_rows) {
      dst[i * cpr + ch] = make_uint4(0, 0, 0, 0);  // the zero row appended after the source rows
    } else if (j >= 0 && j < n_src_rows) {
      dst[i * cpr + ch] = src[j * cpr + ch];
    }                                               // -1 (positions past the counts): untouched
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
                     num_ranks, experts_per_rank, 1, total, permuted_indices, num_tokens_per_expert,
                     (int32_t*)nullptr);
  return launch_status();
}

MOE_API int moe_ep_permute_pad_indices(const int64_t* tokens_per_expert_group, int32_t experts_per_rank,
                                       int32_t num_ranks, int32_t pad_multiple, int64_t total_padded,
                                       int64_t* permuted_indices, int64_t* padded_tokens_per_expert,
                                       int32_t* group_offsets, hipStream_t stream) {
  if (experts_per_rank < 1 || num_ranks < 1 || total_padded < 0 || pad_multiple < 1) return kErrInvalidArgument;
  if ((int64_t)experts_per_rank * num_ranks > kMaxEpSegments) return kErrUnsupportedShape;
  if (!tokens_per_expert_group || (total_padded > 0 && !permuted_indices)) return kErrInvalidArgument;
  int64_t g = (total_padded + 255) / 256;
  if (g > 1024) g = 1024;
  if (g < 1) g = 1;
  hipLaunchKernelGGL(ep_permute_indices_kernel, dim3((int)g), dim3(256), 0, stream, tokens_per_expert_group,
                     num_ranks, experts_per_rank, (int)pad_multiple, total_padded, permuted_indices,
                     padded_tokens_per_expert, group_offsets);
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
