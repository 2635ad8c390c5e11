// Exact log-sum-exp merges.
//
// merge_splits: split-K phase 2.  For query head h with split partials
// (O_s unnormalised, m_s in log2 units, l_s = sum 2^(s - m_s)):
//   M = max_s m_s,  L = sum_s l_s 2^(m_s - M),
//   out = sum_s O_s 2^(m_s - M) / L,  lse = ln 2 * (M + log2 L),
// with the weights 2^(m_s - M) formed once per (head, split).  `out` is
// stored as fp32 or, on request, in the query's dtype (one round to nearest
// even of the fp32 value, what a later Tensor.to(query.dtype) would give);
// lse stays fp32.
// Splits with l_s = 0 (no valid token) contribute nothing: their weight is 0
// and every decode kernel stores their O row as zeros (partial rows are finite
// for finite inputs, so weights multiply them directly); if every split is
// empty, out = 0 and lse = -inf (attention over an empty token set, as
// src/kvssd/backends/reference.py:46-49 returns it).
//
// merge_chunks: the pipeline's running merge of normalised chunk results,
// src/kvssd/attention.py:91-102 (L = logaddexp(La, Lb),
// O = Oa e^(La - L) + Ob e^(Lb - L)), fused into one launch.
#include "decode.hpp"

namespace kvssd {
namespace {

constexpr int kMergeThreads = 256;  // merge_chunks
constexpr int kMaxMergeSplits = 2048;

// One single-wave workgroup per (query head, 16-dim slice): a 32-head decode
// spreads over 256 waves, so every CU pulls a share of the partials.  Splits
// go in batches of 4 OPL (OPL = 64, or 16 when there are at most 64 splits).
// Lane (dim, phase) = (lane / 4, lane % 4) owns the O values of splits
// s = phase (mod 4) of one dim (OPL per batch); lane L owns the (m, l) of
// splits s = L (mod 64) (OPL / 16 per batch).  Every load of a
// batch goes out at once (indices clamped into range, so that no load sits
// under a branch; 32-bit offsets from the uniform base, so that 64 loads in
// flight fit the registers -- 64-bit ones, OFF = uint64_t, only for partials
// beyond 4 GiB): up to 4 OPL splits cost one round trip to memory.
// The batch max and L are wave reductions (DPP and lane reads); the weights
// 2^(m_s - M) go through a per-wave LDS table laid out [phase][j] so that
// each lane reads its 64 weights with 16 vector reads (one wave writes and
// reads it: LDS keeps the order, no barrier); a dim's four phases sit in one
// lane quad and meet by two DPP adds.  A later batch rescales the running
// (M, L, O) exactly.
constexpr int kSliceDims = 16;
constexpr int kPhases = kWave / kSliceDims;  // 4

template <int OPL, typename OFF, typename OT>
__global__ __launch_bounds__(kWave) void merge_splits_kernel(const float* __restrict__ part_o,
                                                            const float* __restrict__ part_ml, int splits,
                                                            int query_heads, int head_dim, OT* __restrict__ out,
                                                            float* __restrict__ lse) {
  constexpr int kBatchSplits = kPhases * OPL;
  constexpr int kOPerLane = OPL;
  constexpr int kMlPerLane = kBatchSplits / kWave;
  __shared__ float sw[kBatchSplits];  // [phase][j]: weight of split phase + 4 j of the batch
  const int h = blockIdx.x;
  const int d0 = blockIdx.y * kSliceDims;
  const int lane = threadIdx.x;
  const int ph = lane % kPhases;
  const int dd = lane / kPhases;
  const bool live = d0 + dd < head_dim;
  const OFF dcol = static_cast<OFF>(live ? d0 + dd : d0);
  const uint8_t* ob = reinterpret_cast<const uint8_t*>(part_o);
  const uint8_t* mb = reinterpret_cast<const uint8_t*>(part_ml);
  const OFF qh = static_cast<OFF>(query_heads), hd = static_cast<OFF>(head_dim);
  // byte offsets: a split index maps to its offset monotonically, so the
  // clamp to the last split is a min on the offset (one add and one min per
  // load, no multiply)
  const OFF o_split = 4u * qh * hd;                         // O bytes per split
  const OFF o_lane = 4u * (static_cast<OFF>(h) * hd + dcol);  // split 0, this lane's dim
  const OFF o_last = static_cast<OFF>(splits - 1) * o_split + o_lane;
  const OFF m_split = 8u * qh;
  const OFF m_last = static_cast<OFF>(splits - 1) * m_split + 8u * static_cast<OFF>(h);
  float big_m = -INFINITY, big_l = 0.0f, acc = 0.0f;
  for (int base = 0; base < splits; base += kBatchSplits) {
    // (m, l) first: the batch max and weights can be formed while the O
    // values are still arriving
    // (the empty asm keeps m0 and o0 opaque: otherwise the compiler folds each
    // load's scalar step back into a per-lane multiply, (base + lane + 64 k) *
    // m_split, one v_mul_lo_u32 per load)
    OFF m0 = static_cast<OFF>(base + lane) * m_split + 8u * static_cast<OFF>(h);
    asm volatile("" : "+v"(m0));
    float2 ml[kMlPerLane];
#pragma unroll
    for (int k = 0; k < kMlPerLane; ++k)
      ml[k] = *reinterpret_cast<const float2*>(mb + min(m0 + static_cast<OFF>(kWave * k) * m_split, m_last));
    OFF o0 = static_cast<OFF>(base + ph) * o_split + o_lane;
    asm volatile("" : "+v"(o0));
    float ov[kOPerLane];
#pragma unroll
    for (int j = 0; j < kOPerLane; ++j)
      ov[j] = *reinterpret_cast<const float*>(ob + min(o0 + static_cast<OFF>(kPhases * j) * o_split, o_last));
    // every load above is issued before any of the math below (the scheduler
    // would otherwise sink the O loads past the (m, l) wait: two round trips)
    __builtin_amdgcn_sched_barrier(0);
    float mv[kMlPerLane], lv[kMlPerLane];
#pragma unroll
    for (int k = 0; k < kMlPerLane; ++k) {
      mv[k] = ml[k].x;
      lv[k] = base + lane + kWave * k < splits ? ml[k].y : 0.0f;
    }
    // M over the non-empty splits seen so far
    float bm = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMlPerLane; ++k) bm = lv[k] > 0.0f ? fmaxf(bm, mv[k]) : bm;
    // (no branch on an empty batch: the O loads must not sink below one; with
    // M = -inf every weight is 0 through the l > 0 guard)
    const float m_new = fmaxf(big_m, wave_max(bm));
    float lsum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMlPerLane; ++k) {
      const float w = lv[k] > 0.0f ? exp2f(mv[k] - m_new) : 0.0f;
      lsum += w * lv[k];
      const int sb = lane + kWave * k;  // split of the batch
      sw[(sb % kPhases) * kOPerLane + sb / kPhases] = w;
    }
    lsum = wave_sum(lsum);
    float osum = 0.0f;
#pragma unroll
    for (int j = 0; j < kOPerLane; j += 4) {
      const float4 w4 = *reinterpret_cast<const float4*>(&sw[ph * kOPerLane + j]);
      osum = __builtin_fmaf(w4.x, ov[j], osum);
      osum = __builtin_fmaf(w4.y, ov[j + 1], osum);
      osum = __builtin_fmaf(w4.z, ov[j + 2], osum);
      osum = __builtin_fmaf(w4.w, ov[j + 3], osum);
    }
    // sum over the 4 phases: the lanes of this lane's quad
    osum += quad_lane<0xB1>(osum);  // quad_perm [1, 0, 3, 2]
    osum += quad_lane<0x4E>(osum);  // quad_perm [2, 3, 0, 1]
    const float rescale = big_l > 0.0f ? exp2f(big_m - m_new) : 0.0f;
    big_l = big_l * rescale + lsum;
    acc = __builtin_fmaf(acc, rescale, osum);
    big_m = m_new;
  }
  if (ph == 0 && live) out[static_cast<long>(h) * head_dim + d0 + dd] = store_cast<OT>(big_l > 0.0f ? acc / big_l : 0.0f);
  if (lane == 0 && blockIdx.y == 0) lse[h] = big_l > 0.0f ? kLn2 * (big_m + log2f(big_l)) : -INFINITY;
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

template <typename OT>
void launch_merge_typed(SplitPartials parts, int splits, int query_heads, int head_dim, OT* out, float* lse,
                        hipStream_t stream) {
  const int slices = (head_dim + kSliceDims - 1) / kSliceDims;
  const dim3 grid(query_heads, slices);
  if (split_partial_bytes(splits, query_heads, head_dim) > 0xFFFFFFFFull)
    hipLaunchKernelGGL((merge_splits_kernel<16, uint64_t, OT>), grid, dim3(kWave), 0, stream, parts.o, parts.ml,
                       splits, query_heads, head_dim, out, lse);
  else if (splits <= kPhases * 16)
    hipLaunchKernelGGL((merge_splits_kernel<16, uint32_t, OT>), grid, dim3(kWave), 0, stream, parts.o, parts.ml,
                       splits, query_heads, head_dim, out, lse);
  else
    hipLaunchKernelGGL((merge_splits_kernel<64, uint32_t, OT>), grid, dim3(kWave), 0, stream, parts.o, parts.ml,
                       splits, query_heads, head_dim, out, lse);
}

int launch_merge_splits(SplitPartials parts, int splits, int query_heads, int head_dim, void* out, int out_dtype,
                        float* lse, hipStream_t stream) {
  if (splits > kMaxMergeSplits) return arg_error("too many splits for the merge kernel");
  switch (out_dtype) {
    case KVSSD_DTYPE_F16:
      launch_merge_typed(parts, splits, query_heads, head_dim, static_cast<_Float16*>(out), lse, stream);
      break;
    case KVSSD_DTYPE_BF16:
      launch_merge_typed(parts, splits, query_heads, head_dim, static_cast<uint16_t*>(out), lse, stream);
      break;
    case KVSSD_DTYPE_F32:
      launch_merge_typed(parts, splits, query_heads, head_dim, static_cast<float*>(out), lse, stream);
      break;
    case KVSSD_DTYPE_F64:
      launch_merge_typed(parts, splits, query_heads, head_dim, static_cast<double*>(out), lse, stream);
      break;
    default:
      return arg_error("unsupported output dtype");
  }
  return hip_status(hipGetLastError(), "merge_splits launch");
}

int launch_merge_chunks(int rows, int dim, float* acc_out, float* acc_lse, const float* out, const float* lse,
                        hipStream_t stream) {
  hipLaunchKernelGGL(merge_chunks_kernel, dim3(rows), dim3(kMergeThreads), 0, stream, dim, acc_out, acc_lse, out,
                     lse);
  return hip_status(hipGetLastError(), "merge_chunks launch");
}

}  // namespace kvssd
