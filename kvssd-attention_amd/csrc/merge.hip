// Exact log-sum-exp merges.
//
// merge_splits: split-K phase 2.  For query head h with split partials
// (O_s unnormalised, m_s in log2 units, l_s = sum 2^(s - m_s)):
//   M = max_s m_s,  L = sum_s l_s 2^(m_s - M),
//   out = sum_s O_s 2^(m_s - M) / L,  lse = ln 2 * (M + log2 L).
// Splits with l_s = 0 (no valid token) contribute nothing; if every split is
// empty, out = 0 and lse = -inf (attention over an empty token set, as
// src/kvssd/backends/reference.py:46-49 returns it).
//
// merge_chunks: the pipeline's running merge of normalised chunk results,
// src/kvssd/attention.py:287-298 (L = logaddexp(La, Lb),
// O = Oa e^(La - L) + Ob e^(Lb - L)), fused into one launch.
#include "decode.hpp"

namespace kvssd {
namespace {

constexpr int kMergeThreads = 256;
constexpr int kMaxSplitWeights = 4096;

// One workgroup per (query head, 32-dim slice).  Phase 1 reduces the global
// max and normaliser over the splits (one split per lane, strided); phase 2
// gives each of the 8 waves' lane groups 32 dims and every 8th split, so each
// load instruction reads 128 contiguous bytes of one split's row, and the 8
// partial sums meet in LDS.
constexpr int kSliceDims = 32;
constexpr int kPhases = kMergeThreads / kSliceDims;  // 8

__global__ __launch_bounds__(kMergeThreads) void merge_splits_kernel(const float* __restrict__ part_o,
                                                                     const float* __restrict__ part_ml, int splits,
                                                                     int query_heads, int head_dim,
                                                                     float* __restrict__ out, float* __restrict__ lse) {
  __shared__ float weight[kMaxSplitWeights];
  __shared__ float red[kMergeThreads / kWave];
  __shared__ float bcast[2];
  __shared__ float partial[kPhases][kSliceDims];
  const int h = blockIdx.x;
  const int d0 = blockIdx.y * kSliceDims;
  const int tid = threadIdx.x;

  // 1) global max over non-empty splits
  float mx = -INFINITY;
  for (int s = tid; s < splits; s += kMergeThreads) {
    const long r = static_cast<long>(s) * query_heads + h;
    if (part_ml[2 * r + 1] > 0.0f) mx = fmaxf(mx, part_ml[2 * r]);
  }
  mx = wave_max(mx);
  if (tid % kWave == 0) red[tid / kWave] = mx;
  __syncthreads();
  if (tid == 0) {
    float m = red[0];
    for (int w = 1; w < kMergeThreads / kWave; ++w) m = fmaxf(m, red[w]);
    bcast[0] = m;
  }
  __syncthreads();
  const float big_m = bcast[0];

  // 2) per-split weights 2^(m_s - M) and the total normaliser
  float lsum = 0.0f;
  for (int s = tid; s < splits; s += kMergeThreads) {
    const long r = static_cast<long>(s) * query_heads + h;
    const float l = part_ml[2 * r + 1];
    const float w = (l > 0.0f) ? exp2f(part_ml[2 * r] - big_m) : 0.0f;
    weight[s] = w;  // splits <= kMaxSplitWeights is checked on the host
    lsum += w * l;
  }
  lsum = wave_sum(lsum);
  __syncthreads();
  if (tid % kWave == 0) red[tid / kWave] = lsum;
  __syncthreads();
  if (tid == 0) {
    float l = 0.0f;
    for (int w = 0; w < kMergeThreads / kWave; ++w) l += red[w];
    bcast[1] = l;
  }
  __syncthreads();
  const float big_l = bcast[1];

  // 3) weighted sum of the unnormalised outputs of this 32-dim slice
  const int dd = tid % kSliceDims;
  const int ph = tid / kSliceDims;
  float acc = 0.0f;
  if (d0 + dd < head_dim) {
    for (int s = ph; s < splits; s += kPhases) {
      const float w = weight[s];
      if (w != 0.0f) acc += w * part_o[(static_cast<long>(s) * query_heads + h) * head_dim + d0 + dd];
    }
  }
  partial[ph][dd] = acc;
  __syncthreads();
  if (tid < kSliceDims && d0 + tid < head_dim) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < kPhases; ++q) sum += partial[q][tid];
    out[static_cast<long>(h) * head_dim + d0 + tid] = big_l > 0.0f ? sum / big_l : 0.0f;
  }
  if (tid == 0 && blockIdx.y == 0) lse[h] = big_l > 0.0f ? kLn2 * (big_m + log2f(big_l)) : -INFINITY;
}

__global__ __launch_bounds__(kMergeThreads) void merge_chunks_kernel(int dim, float* __restrict__ acc_out,
                                                                     float* __restrict__ acc_lse,
                                                                     const float* __restrict__ out,
                                                                     const float* __restrict__ lse) {
  const int r = blockIdx.x;
  const float la = acc_lse[r];
  const float lb = lse[r];
  const float m = fmaxf(la, lb);
  float wa = 0.0f, wb = 0.0f, l = -INFINITY;
  if (m != -INFINITY) {
    const float ea = expf(la - m);
    const float eb = expf(lb - m);
    l = m + logf(ea + eb);
    wa = expf(la - l);
    wb = expf(lb - l);
  }
  for (int dd = threadIdx.x; dd < dim; dd += kMergeThreads) {
    const long i = static_cast<long>(r) * dim + dd;
    const float a = wa != 0.0f ? wa * acc_out[i] : 0.0f;
    const float b = wb != 0.0f ? wb * out[i] : 0.0f;
    acc_out[i] = a + b;
  }
  __syncthreads();  // every lane has read acc_lse[r] before it is replaced
  if (threadIdx.x == 0) acc_lse[r] = l;
}

}  // namespace

int launch_merge_splits(SplitPartials parts, int splits, int query_heads, int head_dim, float* out, float* lse,
                        hipStream_t stream) {
  if (splits > kMaxSplitWeights) return arg_error("too many splits for the merge kernel");
  const int slices = (head_dim + kSliceDims - 1) / kSliceDims;
  hipLaunchKernelGGL(merge_splits_kernel, dim3(query_heads, slices), dim3(kMergeThreads), 0, stream, parts.o,
                     parts.ml, splits, query_heads, head_dim, out, lse);
  return hip_status(hipGetLastError(), "merge_splits launch");
}

int launch_merge_chunks(int rows, int dim, float* acc_out, float* acc_lse, const float* out, const float* lse,
                        hipStream_t stream) {
  hipLaunchKernelGGL(merge_chunks_kernel, dim3(rows), dim3(kMergeThreads), 0, stream, dim, acc_out, acc_lse, out,
                     lse);
  return hip_status(hipGetLastError(), "merge_chunks launch");
}

}  // namespace kvssd
