// Exact log-sum-exp merges.
//
// merge_splits: split-K phase 2.  For query head h with split partials
// (O_s unnormalised, m_s in log2 units, l_s = sum 2^(s - m_s)):
//   M = max_s m_s,  L = sum_s l_s 2^(m_s - M),
//   out = sum_s O_s 2^(m_s - M) / L,  lse = ln 2 * (M + log2 L),
// with the weights 2^(m_s - M) formed once per (head, split).
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
constexpr int kMaxMergeSplits = 2048;

// One workgroup per (query head, 16-dim slice): 8 per head of 128 dims, so a
// 32-head decode spreads over 256 workgroups (every CU pulls a share of the
// partials).  Thread (phase, dim) owns the splits s = phase (mod 16) of one
// dim.  Its first 16 O loads go out together with the workgroup's load of
// every split's (m, l), so the common case (<= 256 splits) costs one round
// trip to memory; the split weights 2^(m_s - M) are formed once, in LDS, and
// the 16 phases meet in LDS at the end.
constexpr int kSliceDims = 16;
constexpr int kPhases = kMergeThreads / kSliceDims;  // 16
constexpr int kBatch = 16;

__global__ __launch_bounds__(kMergeThreads) void merge_splits_kernel(const float* __restrict__ part_o,
                                                                     const float* __restrict__ part_ml, int splits,
                                                                     int query_heads, int head_dim,
                                                                     float* __restrict__ out, float* __restrict__ lse) {
  __shared__ float sw[kMaxMergeSplits];  // m_s, then the weight 2^(m_s - M) (0 for empty splits)
  __shared__ float sl[kMaxMergeSplits];
  __shared__ float red[kMergeThreads / kWave];
  __shared__ float partial[kPhases][kSliceDims];
  const int h = blockIdx.x;
  const int d0 = blockIdx.y * kSliceDims;
  const int tid = threadIdx.x;
  const int dd = tid % kSliceDims;
  const int ph = tid / kSliceDims;
  const bool live = d0 + dd < head_dim;
  const int dcol = live ? d0 + dd : d0;

  float ov[kBatch];
#pragma unroll
  for (int j = 0; j < kBatch; ++j) {
    const int s = ph + kPhases * j;
    ov[j] = s < splits ? part_o[(static_cast<long>(s) * query_heads + h) * head_dim + dcol] : 0.0f;
  }
  float mx = -INFINITY;
  for (int s = tid; s < splits; s += kMergeThreads) {
    const long r = static_cast<long>(s) * query_heads + h;
    const float m = part_ml[2 * r], l = part_ml[2 * r + 1];
    sw[s] = m;
    sl[s] = l;
    if (l > 0.0f) mx = fmaxf(mx, m);
  }
  // M = max over non-empty splits
  mx = wave_max(mx);
  if (tid % kWave == 0) red[tid / kWave] = mx;
  __syncthreads();
  float big_m = red[0];
#pragma unroll
  for (int w = 1; w < kMergeThreads / kWave; ++w) big_m = fmaxf(big_m, red[w]);
  // weights and L = sum_s w_s l_s
  float lsum = 0.0f;
  for (int s = tid; s < splits; s += kMergeThreads) {
    const float l = sl[s];
    const float w = l > 0.0f ? exp2f(sw[s] - big_m) : 0.0f;
    sw[s] = w;
    lsum += w * l;
  }
  lsum = wave_sum(lsum);
  __syncthreads();  // every lane has read red[] before it is reused
  if (tid % kWave == 0) red[tid / kWave] = lsum;
  __syncthreads();  // weights and partial sums visible
  float big_l = 0.0f;
#pragma unroll
  for (int w = 0; w < kMergeThreads / kWave; ++w) big_l += red[w];

  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < kBatch; ++j) {
    const int s = ph + kPhases * j;
    if (s < splits) {
      const float w = sw[s];
      if (w != 0.0f) acc += w * ov[j];
    }
  }
  for (int s = ph + kPhases * kBatch; s < splits; s += kPhases) {
    const float w = sw[s];
    if (w != 0.0f) acc += w * part_o[(static_cast<long>(s) * query_heads + h) * head_dim + dcol];
  }
  partial[ph][dd] = acc;
  __syncthreads();
  if (ph == 0) {
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < kPhases; ++q) sum += partial[q][dd];
    if (live) out[static_cast<long>(h) * head_dim + d0 + dd] = big_l > 0.0f ? sum / big_l : 0.0f;
    if (dd == 0 && blockIdx.y == 0) lse[h] = big_l > 0.0f ? kLn2 * (big_m + log2f(big_l)) : -INFINITY;
  }
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
  if (splits > kMaxMergeSplits) return arg_error("too many splits for the merge kernel");
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
