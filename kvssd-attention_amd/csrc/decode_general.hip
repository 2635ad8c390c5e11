// General fused decode kernel: every shape the reference accepts
// (head_dim <= 256, any group size with head_dim % group_size == 0, INT2/INT4,
// any GQA ratio, any block_tokens), fp32 arithmetic on the VALU.
//
// Semantics: ReferenceAttentionBackend.run (src/kvssd/backends/reference.py:22-50)
// and csrc/fused_decode.cu:12-90 (element addressing :50-56, GQA map :34).
//
// Work split (split-K): workgroup (split, kv_head, head_chunk) owns up to 8
// query heads of one kv head and a contiguous range of attended blocks.  It
// streams 64-token chunks:
//   QK  4 lanes per token, each lane a quarter of the packed row; the lanes'
//       partial dot products meet with two lane-xor shuffles;
//   softmax  one wave per query head updates the running max / sum in log2
//       units (scores pre-multiplied by sm_scale * log2 e);
//   PV  each lane owns (head, dim) outputs and accumulates p * v over the
//       chunk, reading codes and scales straight from L2 (adjacent lanes hold
//       adjacent dims, so a wave reads one packed row contiguously).
// The split's unnormalised (O, m, l) go to the workspace; merge.hip finishes.
#include "decode.hpp"

namespace kvssd {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 64;
constexpr int kMaxHeads = 8;
constexpr int kMaxDim = 256;
constexpr int kOutPerThread = kMaxHeads * kMaxDim / kThreads;  // 8

struct GeneralParams {
  const void* query;
  const uint8_t* pk;
  const uint8_t* pv;
  const uint16_t* sk;
  const uint16_t* sv;
  const int32_t* valid;
  const int32_t* table;
  float* part_o;
  float* part_ml;
  int query_heads, kv_heads, head_dim, block_tokens, groups, group_size, packed_dim, num_blocks;
  int units, blocks_per_split, heads_per_chunk, head_chunks;
  float scale_log2;  // sm_scale * log2(e)
};

template <typename QT, int BITS>
__global__ __launch_bounds__(kThreads) void decode_general_kernel(GeneralParams p) {
  constexpr int kPer = 8 / BITS;
  constexpr int kMask = (1 << BITS) - 1;
  constexpr int kMid = 1 << (BITS - 1);

  __shared__ float q_s[kMaxHeads][kMaxDim];
  __shared__ float prob[kMaxHeads][kChunk];
  __shared__ float m_run[kMaxHeads], l_run[kMaxHeads], alpha_s[kMaxHeads];

  const int tid = threadIdx.x;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y / p.head_chunks;
  const int chunk_id = blockIdx.y % p.head_chunks;
  const int gq = p.query_heads / p.kv_heads;
  const int h0 = kvh * gq + chunk_id * p.heads_per_chunk;
  const int nh = min(p.heads_per_chunk, gq - chunk_id * p.heads_per_chunk);
  const int d = p.head_dim;

  for (int i = tid; i < nh * d; i += kThreads) q_s[i / d][i % d] = load_query<QT>(p.query, (h0 + i / d) * d + i % d);
  if (tid < kMaxHeads) {
    m_run[tid] = -INFINITY;
    l_run[tid] = 0.0f;
  }
  float acc[kOutPerThread];
#pragma unroll
  for (int k = 0; k < kOutPerThread; ++k) acc[k] = 0.0f;
  __syncthreads();

  const int u_begin = split * p.blocks_per_split;
  const int u_end = min(p.units, u_begin + p.blocks_per_split);
  const int lane_tok = tid / 4;
  const int part = tid % 4;
  const int wave = tid / kWave;
  const int lane = tid % kWave;

  for (int u = u_begin; u < u_end; ++u) {
    const int blk = p.table ? p.table[u] : u;
    if (blk < 0 || blk >= p.num_blocks) continue;  // ids are checked on the host; never read out of bounds
    const int vb = clamp_valid(p.valid[blk], p.block_tokens);
    for (int c0 = 0; c0 < vb; c0 += kChunk) {
      const int n = min(kChunk, vb - c0);
      // ---- QK: lane group of 4 per token
      float sc[kMaxHeads];
#pragma unroll
      for (int hh = 0; hh < kMaxHeads; ++hh) sc[hh] = 0.0f;
      if (lane_tok < n) {
        const long row = (static_cast<long>(blk) * p.block_tokens + c0 + lane_tok) * p.kv_heads + kvh;
        const uint8_t* krow = p.pk + row * p.packed_dim;
        const uint16_t* srow = p.sk + row * p.groups;
        for (int b = part; b < p.packed_dim; b += 4) {
          const unsigned byte = krow[b];
#pragma unroll
          for (int i = 0; i < kPer; ++i) {
            const int dd = b * kPer + i;
            const float kval = static_cast<float>(static_cast<int>((byte >> (i * BITS)) & kMask) - kMid) *
                               half_bits_to_float(srow[dd / p.group_size]);
#pragma unroll
            for (int hh = 0; hh < kMaxHeads; ++hh)
              if (hh < nh) sc[hh] += q_s[hh][dd] * kval;
          }
        }
      }
#pragma unroll
      for (int hh = 0; hh < kMaxHeads; ++hh) {
        sc[hh] += __shfl_xor(sc[hh], 1, kWave);
        sc[hh] += __shfl_xor(sc[hh], 2, kWave);
      }
      if (part == 0) {
#pragma unroll
        for (int hh = 0; hh < kMaxHeads; ++hh) prob[hh][lane_tok] = sc[hh] * p.scale_log2;
      }
      __syncthreads();
      // ---- online softmax: one wave per head, one lane per token
      for (int hh = wave; hh < nh; hh += kThreads / kWave) {
        const float s = lane < n ? prob[hh][lane] : -INFINITY;
        const float mx = wave_max(s);
        const float m_old = m_run[hh];
        const float m_new = fmaxf(m_old, mx);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2f(m_old - m_new);
        const float pr = lane < n ? exp2f(s - m_new) : 0.0f;
        const float sum = wave_sum(pr);
        prob[hh][lane] = pr;
        if (lane == 0) {
          l_run[hh] = l_run[hh] * alpha + sum;
          m_run[hh] = m_new;
          alpha_s[hh] = alpha;
        }
      }
      __syncthreads();
      // ---- PV: each lane owns outputs o = tid + k * kThreads
#pragma unroll
      for (int k = 0; k < kOutPerThread; ++k) {
        const int o = tid + k * kThreads;
        if (o < nh * d) {
          const int hh = o / d;
          const int dd = o % d;
          float a = acc[k] * alpha_s[hh];
          const long row0 = (static_cast<long>(blk) * p.block_tokens + c0) * p.kv_heads + kvh;
          const int byte_off = dd / kPer;
          const int shift = (dd % kPer) * BITS;
          const int grp = dd / p.group_size;
          for (int j = 0; j < n; ++j) {
            const long row = row0 + static_cast<long>(j) * p.kv_heads;
            const int code = (p.pv[row * p.packed_dim + byte_off] >> shift) & kMask;
            const float v = static_cast<float>(code - kMid) * half_bits_to_float(p.sv[row * p.groups + grp]);
            a += prob[hh][j] * v;
          }
          acc[k] = a;
        }
      }
      __syncthreads();
    }
  }
  // ---- unnormalised partial of this split
#pragma unroll
  for (int k = 0; k < kOutPerThread; ++k) {
    const int o = tid + k * kThreads;
    if (o < nh * d) {
      const int hh = o / d;
      p.part_o[(static_cast<long>(split) * p.query_heads + h0 + hh) * d + o % d] = acc[k];
    }
  }
  if (tid < nh) {
    const long r = static_cast<long>(split) * p.query_heads + h0 + tid;
    p.part_ml[2 * r] = m_run[tid];
    p.part_ml[2 * r + 1] = l_run[tid];
  }
}

template <typename QT>
int launch_typed(const GeneralParams& prm, dim3 grid, int bits, hipStream_t s) {
  if (bits == 4)
    hipLaunchKernelGGL((decode_general_kernel<QT, 4>), grid, dim3(kThreads), 0, s, prm);
  else
    hipLaunchKernelGGL((decode_general_kernel<QT, 2>), grid, dim3(kThreads), 0, s, prm);
  return hip_status(hipGetLastError(), "decode_general launch");
}

}  // namespace

SplitPlan plan_splits(const kvssd_decode_desc& d, int units) {
  // about 1024 (kv head, split) work items: one resident round of the
  // matrix-core kernel (4 single-wave workgroups per CU on a 256-CU part, each
  // streaming its blocks with loads one sub-block ahead); the general kernel
  // runs 1024+ four-wave workgroups.  2048 where the staged kernel gives each
  // workgroup all 8 kv heads of a row: 256 workgroups either way.
  const long items = staged_wide(d, units) ? 2048 : 1024;
  long per = (static_cast<long>(units) * d.kv_heads + items - 1) / items;
  SplitPlan plan{};
  plan.blocks_per_split = static_cast<int>(per < 1 ? 1 : per);
  plan.splits = (units + plan.blocks_per_split - 1) / plan.blocks_per_split;
  return plan;
}

int launch_general(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts) {
  const kvssd_decode_desc& d = a.desc;
  const int gq = d.query_heads / d.kv_heads;
  const int heads_per_chunk = gq < kMaxHeads ? gq : kMaxHeads;
  const int head_chunks = (gq + heads_per_chunk - 1) / heads_per_chunk;
  GeneralParams prm{};
  prm.query = a.query;
  prm.pk = a.packed_k;
  prm.pv = a.packed_v;
  prm.sk = a.scales_k;
  prm.sv = a.scales_v;
  prm.valid = a.valid;
  prm.table = a.table;
  prm.part_o = parts.o;
  prm.part_ml = parts.ml;
  prm.query_heads = d.query_heads;
  prm.kv_heads = d.kv_heads;
  prm.head_dim = d.head_dim;
  prm.block_tokens = d.block_tokens;
  prm.num_blocks = d.num_blocks;
  prm.group_size = d.group_size;
  prm.groups = d.head_dim / d.group_size;
  prm.packed_dim = d.head_dim * d.bits / 8;
  prm.units = a.units;
  prm.blocks_per_split = plan.blocks_per_split;
  prm.heads_per_chunk = heads_per_chunk;
  prm.head_chunks = head_chunks;
  prm.scale_log2 = static_cast<float>(d.sm_scale) * kLog2e;
  dim3 grid(plan.splits, d.kv_heads * head_chunks);
  switch (d.query_dtype) {
    case KVSSD_DTYPE_F16:
      return launch_typed<_Float16>(prm, grid, d.bits, a.stream);
    case KVSSD_DTYPE_BF16:
      return launch_typed<uint16_t>(prm, grid, d.bits, a.stream);
    case KVSSD_DTYPE_F32:
      return launch_typed<float>(prm, grid, d.bits, a.stream);
    case KVSSD_DTYPE_F64:
      return launch_typed<double>(prm, grid, d.bits, a.stream);
    default:
      return arg_error("unsupported query dtype");
  }
}

}  // namespace kvssd
