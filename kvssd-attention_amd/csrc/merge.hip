// Exact log-sum-exp merges.
//
// merge_splits: split-K phase 2.  For query head h with split partials
// (O_s unnormalised, m_s in log2 units, l_s = sum 2^(s - m_s)):
//   M = max_s m_s,  L = sum_s l_s 2^(m_s - M),
//   out = sum_s O_s 2^(m_s - M) / L,  lse = ln 2 * (M + log2 L),
// evaluated as a running fold (m, l, o) <- (max, rescaled sums), which gives
// the same M and the same terms.
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

// One workgroup per (query head, 32-dim slice); thread (phase, dim) folds the
// splits s = phase (mod 8) into a running (m, l, o) with the online rescaling
// (loads 16 splits at a time so their latencies overlap), then the 8 phases
// meet in LDS.  One pass over the partials, no second round trip for the
// global max.
constexpr int kSliceDims = 32;
constexpr int kPhases = kMergeThreads / kSliceDims;  // 8
constexpr int kBatch = 16;

__device__ __forceinline__ void fold(float& m, float& l, float& o, float ms, float ls, float os) {
  if (ls > 0.0f) {
    const float mn = fmaxf(m, ms);
    const float a = exp2f(m - mn);  // m = -inf on the first fold: a = 0
    const float b = exp2f(ms - mn);
    o = o * a + os * b;
    l = l * a + ls * b;
    m = mn;
  }
}

__global__ __launch_bounds__(kMergeThreads) void merge_splits_kernel(const float* __restrict__ part_o,
                                                                     const float* __restrict__ part_ml, int splits,
                                                                     int query_heads, int head_dim,
                                                                     float* __restrict__ out, float* __restrict__ lse) {
  __shared__ float sm[kPhases][kSliceDims], sl[kPhases][kSliceDims], so[kPhases][kSliceDims];
  const int h = blockIdx.x;
  const int d0 = blockIdx.y * kSliceDims;
  const int dd = threadIdx.x % kSliceDims;
  const int ph = threadIdx.x / kSliceDims;
  const bool live = d0 + dd < head_dim;
  const int dcol = live ? d0 + dd : d0;
  float m = -INFINITY, l = 0.0f, o = 0.0f;
  int s = ph;
  for (; s + (kBatch - 1) * kPhases < splits; s += kBatch * kPhases) {
    float ms[kBatch], ls[kBatch], os[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const long r = static_cast<long>(s + b * kPhases) * query_heads + h;
      ms[b] = part_ml[2 * r];
      ls[b] = part_ml[2 * r + 1];
      os[b] = part_o[r * head_dim + dcol];
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) fold(m, l, o, ms[b], ls[b], os[b]);
  }
  for (; s < splits; s += kPhases) {
    const long r = static_cast<long>(s) * query_heads + h;
    fold(m, l, o, part_ml[2 * r], part_ml[2 * r + 1], part_o[r * head_dim + dcol]);
  }
  sm[ph][dd] = m;
  sl[ph][dd] = l;
  so[ph][dd] = o;
  __syncthreads();
  if (ph == 0) {
#pragma unroll
    for (int q = 1; q < kPhases; ++q) fold(m, l, o, sm[q][dd], sl[q][dd], so[q][dd]);
    if (live) out[static_cast<long>(h) * head_dim + d0 + dd] = l > 0.0f ? o / l : 0.0f;
    if (dd == 0 && blockIdx.y == 0) lse[h] = l > 0.0f ? kLn2 * (m + log2f(l)) : -INFINITY;
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
