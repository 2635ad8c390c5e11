// Matrix-core fused decode kernel for gfx950: head_dim 128, group_size 32,
// INT4 or INT2 codes, up to 8 query heads per kv head, block_tokens % 128 == 0.
//
// Same semantics as the general kernel (ReferenceAttentionBackend.run,
// src/kvssd/backends/reference.py:22-50; element addressing of
// csrc/fused_decode.cu:50-56).  One wave owns (kv head, range of blocks) and
// streams 128-token sub-blocks; the packed rows of the kv head are read once
// and shared by all its query heads -- or, with more than 4 query heads per kv
// head on a grid small enough to be resident at once, one wave per (kv head,
// query quad, range of blocks), each reading the rows (the second one mostly
// from L2) for half the math.
//
// Code -> fp16 without a dequantised tensor: a code c placed in the mantissa of
// 1.0 gives v = 1 + c/F (F = 64 for INT4, 4 for INT2; common.hpp), and
// (c - mid) = F (v - OFF) with OFF = 1 + mid/F.
//
// QK (v_mfma_f32_16x16x32_f16, 4 per 16-token tile and query quad):
//   A = query, rows (h', g') = 4 heads x 4 groups, each row holding head h'
//       masked to group g' (zero elsewhere); B = K codes as v, columns = the 16
//       tokens of the tile.  Lane l loads 16 B (INT4) / 8 B (INT2) of token
//       l%16's row at chunk l/16, i.e. group l/16 of that token; MFMA m takes
//       word m (INT4) / a half of word m/2 (INT2).  C starts at
//       -OFF * sum_{d in g'} q[h',d], so C[(h',g'),t] = sum_{d in g'} q (c-mid)/F.
//   Lane l ends with the 4 groups of head l/16, token l%16, and forms
//   s = F * sm_scale * log2(e) * sum_g scale_k[t,g] * C[g] in registers.
// softmax: exact per sub-block max (16-lane row reduction), running (m, l) in
//   log2 units; p = 2^(s - m), m including a per-sub-block power of two e set
//   by the sub-block's largest V scale so that W below stays in fp16's normal
//   range (common.hpp).
// PV (v_mfma_f32_16x16x32_f16, per 32-token K step, 8 dim tiles, per quad):
//   A = V^T codes as v: a 16x16 nibble transpose read (ds_read_b64_tr_b4) of
//       the sub-block's V rows staged in LDS gives lane l one dim across 16
//       tokens (two K steps' worth); INT2 nibbles carry two dims each (even
//       and odd tiles).
//   B = W, columns (h'', g'') = 4 heads x 4 groups: W[t,(h,g)] = p[h,t] *
//       scale_v[t,g] in fp16, written by the QK lanes into LDS and read back
//       16 B per lane.  Only the column whose group owns a tile's dims is kept;
//       out = F * (C - OFF * sum_t W), the sum taken from the same fp16 W.
// Software pipelining: the next sub-block's loads (K, V, both scale rows) go
// out into a second register stage before the current sub-block computes, so
// every wave keeps ~18 KB in flight while its MFMAs and VALU run.
// Token <-> MFMA K-slot map (shared by A and B): K step k, lane group q,
//   slot s -> token 16*dimperm(s) + 4q + k, dimperm(s) = (s>>1) + 4(s&1)
//   (the order the magic unpack leaves nibbles in).  The tr read row r of
//   lane group q for K-step pair kp is token 16(r%8) + 4q + 2kp + r/8.
// LDS layouts (conflict-free for the tr reads, 64 banks):
//   INT4 V: token T, 8-byte unit n at T*64 + 8*(n ^ (T>>4)).
//   INT2 V: row R = (T & ~15) | ((T & 15) ^ (T >> 4)), unit n at
//           R*32 + 8*(n ^ 2*(T&1)).
//   W: [quad][h*4+g][slot], rows of 272 B (256 B + 16 B pad), slot for token
//      16*tau + t at 32*(t%4) + 8*(t/4) + dimperm^-1(tau).
// Non-fp16 queries are normalised per head by a power of two, fp32 and fp64
// ones split into hi + lo fp16 parts (two MFMAs per step; bf16 values fit one
// part); the power of two returns in the score scale, so the products stay
// exact.
#include <type_traits>

#include "decode.hpp"

namespace kvssd {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kSub = 128;           // tokens per sub-block
constexpr int kTiles = kSub / 16;   // QK tiles per sub-block
constexpr int kWRow = 272;          // bytes per W row: 128 fp16 slots + 16 B pad
// one-wave workgroups resident at once at one wave per SIMD (256 CUs x 4 SIMDs;
// the kernel's registers allow no more)
constexpr long kMfmaResidentWaves = 1024;

struct MfmaParams {
  const void* query;
  const uint8_t* pk;
  const uint8_t* pv;
  const uint16_t* sk;
  const uint16_t* sv;
  const int32_t* valid;
  const int32_t* table;
  float* part_o;
  float* part_ml;
  int query_heads, kv_heads, block_tokens, num_blocks, units, splits, blocks_per_split, gq;
  float scale_log2;  // sm_scale * log2(e)
};

__device__ __forceinline__ int dimperm(int s) { return (s >> 1) + 4 * (s & 1); }

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c, 0,
                                                0, 0);
}

__device__ __forceinline__ uint32_t pack_half2(_Float16 lo, _Float16 hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

// dim of MFMA m's slot s for lane group q (K operand of the QK product)
template <int BITS>
__device__ __forceinline__ int qk_dim(int m, int q, int s) {
  if (BITS == 4) return 32 * q + 8 * m + dimperm(s);
  return 32 * q + 16 * (m >> 1) + 4 * (m & 1) + (s >> 1) + 8 * (s & 1);
}

// B operand of QK MFMA m from the lane's loaded K chunk
template <int BITS>
__device__ __forceinline__ u32x4 k_operand(const u32x4& raw, int m) {
  u32x4 out;
  if (BITS == 4) {
    uint32_t w[4];
    unpack_int4_f16(raw[m], w);
    out = u32x4{w[0], w[1], w[2], w[3]};
  } else {
    uint32_t w[8];
    unpack_int2_f16(raw[m >> 1], w);
    const int o = 4 * (m & 1);
    out = u32x4{w[o], w[o + 1], w[o + 2], w[o + 3]};
  }
  return out;
}

// INT2 nibble-transposed word -> fp16 (row j, row j+4) pairs of one code lane
// (parity 0: even dim, bits 4r..4r+1; parity 1: odd dim, bits 4r+2..4r+3).
__device__ __forceinline__ u32x4 int2_tr_operand(uint32_t x, int parity) {
  const uint32_t m = kMaskInt2;
  u32x4 out;
  if (parity == 0) {
    out[0] = and_or(x << 8, m, kF16One2);
    out[1] = and_or(x << 4, m, kF16One2);
    out[2] = and_or(x, m, kF16One2);
    out[3] = and_or(x >> 4, m, kF16One2);
  } else {
    out[0] = and_or(x << 6, m, kF16One2);
    out[1] = and_or(x << 2, m, kF16One2);
    out[2] = and_or(x >> 2, m, kF16One2);
    out[3] = and_or(x >> 6, m, kF16One2);
  }
  return out;
}

// ds_read_b64_tr_b4 at a byte offset of a __shared__ array: within each group
// of 16 lanes, lane j receives nibble j of the 8 bytes every lane of the group
// addressed, lane r's nibble landing in bits 4r..4r+3 (a 16x16 nibble transpose)
__device__ __forceinline__ i32x2 lds_read_tr4(const uint8_t* lds, int offset) {
  typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
  return __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2*)(lds + offset));
}

template <typename QT>
__device__ __forceinline__ float query_at(const MfmaParams& p, int head, int d) {
  return load_query<QT>(p.query, head * 128 + d);
}

// ------------------------------------------------------------------ stages
// Registers of one 128-token sub-block's loads (INT2 uses the first two words).
struct Stage {
  u32x4 k[kTiles], v[kTiles];
  u32x2 sk[kTiles], sv[kTiles];
};

// Position in the wave's work: unit u (attended block), its block id, its
// clamped valid count and the current sub-block start.
struct Cursor {
  int u, blk, vb, sb0;
};

// Advance to the next sub-block holding at least one valid token; false at the
// end of the wave's units.  All values are wave-uniform.
__device__ __forceinline__ bool next_sub(Cursor& c, const MfmaParams& p, int u_end) {
  c.sb0 += kSub;
  while (c.sb0 >= c.vb) {
    if (++c.u >= u_end) return false;
    const int blk = p.table ? p.table[c.u] : c.u;
    c.blk = blk;
    c.vb = (blk < 0 || blk >= p.num_blocks) ? 0 : clamp_valid(p.valid[blk], p.block_tokens);  // host-checked ids
    c.sb0 = 0;
  }
  return true;
}

template <int BITS>
__device__ __forceinline__ void issue_loads(Stage& st, const MfmaParams& p, const Cursor& c, int kvh, int li, int lq) {
  constexpr int PD = 128 * BITS / 8;
  const long tok0 = static_cast<long>(c.blk) * p.block_tokens + c.sb0;
#pragma unroll
  for (int tau = 0; tau < kTiles; ++tau) {
    const long row = (tok0 + 16 * tau + li) * p.kv_heads + kvh;
    if (BITS == 4) {
      st.k[tau] = *reinterpret_cast<const u32x4*>(p.pk + row * PD + 16 * lq);
      st.v[tau] = *reinterpret_cast<const u32x4*>(p.pv + row * PD + 16 * lq);
    } else {
      const u32x2 k2 = *reinterpret_cast<const u32x2*>(p.pk + row * PD + 8 * lq);
      const u32x2 v2 = *reinterpret_cast<const u32x2*>(p.pv + row * PD + 8 * lq);
      st.k[tau] = u32x4{k2[0], k2[1], 0u, 0u};
      st.v[tau] = u32x4{v2[0], v2[1], 0u, 0u};
    }
    st.sk[tau] = *reinterpret_cast<const u32x2*>(p.sk + row * 4);
    st.sv[tau] = *reinterpret_cast<const u32x2*>(p.sv + row * 4);
  }
}

// Running state of one query quad.
struct QuadState {
  float m_run, l_run, wsum;
  f32x4 acc[8];
};

template <int BITS, int QUADS, int QSPLIT>
__device__ __forceinline__ void process(const Stage& st, const Cursor& c, uint8_t* v_lds, uint8_t* w_lds,
                                        const u32x4 (&qa)[QUADS][QSPLIT][4], const f32x4 (&qcorr)[QUADS],
                                        const float (&kscale)[QUADS], QuadState (&qs)[QUADS], int li, int lq) {
  __syncthreads();  // the previous sub-block's LDS reads are done
  // ------------------------------------------------------------ V rows -> LDS
#pragma unroll
  for (int tau = 0; tau < kTiles; ++tau) {
    const int t = 16 * tau + li;
    if (BITS == 4) {
      const u32x4 v = st.v[tau];
      const u32x4 w = (tau & 1) ? u32x4{v[2], v[3], v[0], v[1]} : v;
      *reinterpret_cast<u32x4*>(v_lds + t * 64 + 16 * (lq ^ (tau >> 1))) = w;
    } else {
      const int r = (t & ~15) | ((t & 15) ^ tau);
      const int pos = lq ^ (2 * (t & 1));
      *reinterpret_cast<u32x2*>(v_lds + r * 32 + 8 * pos) = u32x2{st.v[tau][0], st.v[tau][1]};
    }
  }
  // -------------------------------------------------------------------- QK
  float score[QUADS][kTiles];
#pragma unroll
  for (int tau = 0; tau < kTiles; ++tau) {
    u32x4 b[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) b[m] = k_operand<BITS>(st.k[tau], m);
    const uint32_t s01 = st.sk[tau][0], s23 = st.sk[tau][1];
    const float sk0 = half_bits_to_float(static_cast<uint16_t>(s01 & 0xFFFFu));
    const float sk1 = half_bits_to_float(static_cast<uint16_t>(s01 >> 16));
    const float sk2 = half_bits_to_float(static_cast<uint16_t>(s23 & 0xFFFFu));
    const float sk3 = half_bits_to_float(static_cast<uint16_t>(s23 >> 16));
    const bool ok = c.sb0 + 16 * tau + li < c.vb;
#pragma unroll
    for (int quad = 0; quad < QUADS; ++quad) {
      f32x4 cc = qcorr[quad];
#pragma unroll
      for (int sp = 0; sp < QSPLIT; ++sp)
#pragma unroll
        for (int m = 0; m < 4; ++m) cc = mfma16(qa[quad][sp][m], b[m], cc);
      const float sc = (sk0 * cc[0] + sk1 * cc[1] + sk2 * cc[2] + sk3 * cc[3]) * kscale[quad];
      score[quad][tau] = ok ? sc : -INFINITY;
    }
  }
  // --------------------------------------------------------------- softmax
  // the sub-block's V-scale exponent (wave-uniform; every lane row holds the
  // same tokens): W = 2^(s - (m + e)) scale_v stays in fp16's normal range
  uint32_t smax = 0u;
#pragma unroll
  for (int tau = 0; tau < kTiles; ++tau) {
    const uint32_t b = abs_max_bits(st.sv[tau][0], st.sv[tau][1]);
    smax = c.sb0 + 16 * tau + li < c.vb && b > smax ? b : smax;
  }
  const float e_v = static_cast<float>(wave_scale_exp(smax));
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    float mx = score[quad][0];
#pragma unroll
    for (int tau = 1; tau < kTiles; ++tau) mx = fmaxf(mx, score[quad][tau]);
    mx = row_max16(mx) + e_v;  // the running reference: max of (sub-block max + e)
    const float m_new = fmaxf(qs[quad].m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(qs[quad].m_run - m_new);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    qs[quad].m_run = m_new;
    float psum = 0.0f;
    _Float16 w[4][kTiles];
#pragma unroll
    for (int tau = 0; tau < kTiles; ++tau) {
      // masked tokens: score -inf gives p = 0, and their scales (possibly
      // garbage padding) are replaced by 0 with a select, never a branch
      const bool ok = score[quad][tau] != -INFINITY;
      const float pr = __builtin_amdgcn_exp2f(score[quad][tau] - m_use);
      psum += pr;
      const uint32_t s01 = ok ? st.sv[tau][0] : 0u;
      const uint32_t s23 = ok ? st.sv[tau][1] : 0u;
      w[0][tau] = static_cast<_Float16>(pr * half_bits_to_float(static_cast<uint16_t>(s01 & 0xFFFFu)));
      w[1][tau] = static_cast<_Float16>(pr * half_bits_to_float(static_cast<uint16_t>(s01 >> 16)));
      w[2][tau] = static_cast<_Float16>(pr * half_bits_to_float(static_cast<uint16_t>(s23 & 0xFFFFu)));
      w[3][tau] = static_cast<_Float16>(pr * half_bits_to_float(static_cast<uint16_t>(s23 >> 16)));
    }
    qs[quad].l_run = qs[quad].l_run * alpha + psum;
    // W rows: slot 32*(t%4) + 8*(t/4) + s holds tile dimperm(s)
    uint8_t* wbase = w_lds + quad * 16 * kWRow + (32 * (li & 3) + 8 * (li >> 2)) * 2;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x4 v = u32x4{pack_half2(w[g][0], w[g][4]), pack_half2(w[g][1], w[g][5]), pack_half2(w[g][2], w[g][6]),
                            pack_half2(w[g][3], w[g][7])};
      *reinterpret_cast<u32x4*>(wbase + (lq * 4 + g) * kWRow) = v;
    }
    // rescale the PV state of column head li/4 by that head's alpha
    const float a_pv = __shfl(alpha, (li >> 2) << 4, kWave);
    if (__any(a_pv != 1.0f)) {
      qs[quad].wsum *= a_pv;
#pragma unroll
      for (int n = 0; n < 8; ++n) qs[quad].acc[n] *= a_pv;
    }
  }
  __syncthreads();  // V and W tiles visible to every lane
  // -------------------------------------------------------------------- PV
#pragma unroll
  for (int kp = 0; kp < 2; ++kp) {
    u32x4 wb[QUADS][2];
#pragma unroll
    for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int k = 2 * kp + kk;
        wb[quad][kk] = *reinterpret_cast<const u32x4*>(w_lds + quad * 16 * kWRow + li * kWRow + (32 * k + 8 * lq) * 2);
      }
    // tr row of this lane: token 16*(r%8) + 4q + 2kp + r/8 with r = li
    const int tt = 16 * (li & 7) + 4 * lq + 2 * kp + (li >> 3);
    if (BITS == 4) {
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const i32x2 tr = lds_read_tr4(v_lds, tt * 64 + 8 * (n ^ (li & 7)));
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          uint32_t wv[4];
          unpack_int4_f16(static_cast<uint32_t>(tr[kk]), wv);
          const u32x4 a = u32x4{wv[0], wv[1], wv[2], wv[3]};
#pragma unroll
          for (int quad = 0; quad < QUADS; ++quad) qs[quad].acc[n] = mfma16(a, wb[quad][kk], qs[quad].acc[n]);
        }
      }
    } else {
      const int r = (tt & ~15) | ((tt & 15) ^ (tt >> 4));
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const i32x2 tr = lds_read_tr4(v_lds, r * 32 + 8 * (n ^ (2 * (li >> 3))));
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int par = 0; par < 2; ++par) {
            const u32x4 a = int2_tr_operand(static_cast<uint32_t>(tr[kk]), par);
#pragma unroll
            for (int quad = 0; quad < QUADS; ++quad)
              qs[quad].acc[2 * n + par] = mfma16(a, wb[quad][kk], qs[quad].acc[2 * n + par]);
          }
      }
    }
    // column sums of W over this lane's K slots (the fp16 values the MFMA saw);
    // plain converts and adds: v_dot2c_f32_f16 against (1, 1) returned wrong
    // sums in testing, so it is not used here
#pragma unroll
    for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t x = wb[quad][kk][j];
          qs[quad].wsum += half_bits_to_float(static_cast<uint16_t>(x & 0xFFFFu)) +
                           half_bits_to_float(static_cast<uint16_t>(x >> 16));
        }
  }
}

template <int BITS, int QUADS, int QSPLIT, typename QT>
__global__ __launch_bounds__(64) void decode_mfma_kernel(const void* query, const uint8_t* pk, const uint8_t* pv,
                                                        const uint16_t* sk, const uint16_t* sv, uint32_t heads,
                                                        int block_tokens, int blocks_per_split, int units_total,
                                                        DecodeTail r) {
  const MfmaParams p{query,        pk,
                     pv,           sk,
                     sv,           r.valid,
                     r.table,      r.part_o,
                     r.part_ml,    r.query_heads,
                     static_cast<int>(heads & 0xFFFFu), block_tokens,
                     r.num_blocks, units_total,
                     r.splits,     blocks_per_split,
                     static_cast<int>((heads >> 16) & 0xFFu), r.scale_log2};
  const bool has_table = (heads & kHasTable) != 0;
  constexpr float F = kUnpackScale<BITS>;
  constexpr float OFF = kUnpackOffset<BITS>;
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[kSub * 128 * BITS / 8];
  __shared__ __attribute__((aligned(16))) uint8_t w_lds[QUADS * 16 * kWRow];

  const int lane = threadIdx.x;
  const int li = lane & 15;
  const int lq = lane >> 4;

  // XCD-aware placement: consecutive workgroup ids go to different XCDs; the
  // kv heads of one split (which share 128-byte lines of the packed rows) get
  // ids 8 apart, i.e. the same XCD and its L2.  With a workgroup per query
  // quad (kQuadPerGroup; QUADS == 1, more than 4 query heads per kv head) the
  // two quads of a kv head come next to each other in that order, so the
  // second reads the kv head's codes from the same L2.
  const int bid = blockIdx.x;
  const int xcd = bid & 7;
  const int rest = bid >> 3;
  const int qshift = (heads & kQuadPerGroup) ? 1 : 0;
  const int slots = p.kv_heads << qshift;  // workgroups per split
  const int slot = rest % slots;
  const int kvh = slot >> qshift;
  const int quad0 = slot & qshift;  // this workgroup's first query quad
  const int split = (rest / slots) * 8 + xcd;
  const int u_begin = split * p.blocks_per_split;
  // padding ids of the last round (splits = ceil(units / blocks_per_split))
  if (u_begin >= p.units) return;
  const int u_end = min(p.units, u_begin + p.blocks_per_split);
  // this workgroup's query heads: gqw heads from head0, i.e. query quads
  // quad0 .. quad0 + QUADS - 1 of the kv head (the last one possibly partial)
  const int head0 = kvh * p.gq + 4 * quad0;
  const int gqw = min(p.gq - 4 * quad0, 4 * QUADS);

  // The first sub-block's loads go out before the query set-up.  Without a
  // block table they go out at entry, before the first block's valid count is
  // known (a round trip): the split's first block, its first 128 tokens (in
  // bounds: u_begin < units = num_blocks).  If that sub-block holds no valid
  // token they are simply replaced.
  Stage s0, s1;
  const bool spec = !has_table;
  if (spec) issue_loads<BITS>(s0, p, Cursor{u_begin, u_begin, 0, 0}, kvh, li, lq);
  // the non-preloaded arguments, in SGPRs from here on (they stay live, so no
  // register of theirs is reused before this point)
  asm volatile("" ::"s"(r.valid), "s"(r.table), "s"(r.part_o), "s"(r.part_ml), "s"(r.query_heads),
               "s"(r.num_blocks), "s"(r.scale_log2), "s"(r.splits));
  Cursor cur{u_begin - 1, 0, 0, 0};
  bool have0 = next_sub(cur, p, u_end);
  Cursor c0 = cur;
  if (have0 && !(spec && c0.blk == u_begin && c0.sb0 == 0)) issue_loads<BITS>(s0, p, c0, kvh, li, lq);

  // ---------------------------------------------------------------- query
  constexpr bool kNormalise = !std::is_same<QT, _Float16>::value;
  u32x4 qa[QUADS][QSPLIT][4];
  f32x4 qcorr[QUADS];
  float kscale[QUADS];
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    // per-head power-of-two normaliser (exact); fp16 queries are used as is
    const int hrow = quad * 4 + lq;  // head of this lane's QK row
    const int hrow_c = hrow < gqw ? hrow : gqw - 1;
    float e_row = 0.0f;
    if (kNormalise) {
      float mx = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(query_at<QT>(p, head0 + hrow_c, 8 * li + i)));
      mx = row_max16(mx);
      int ex = 0;
      if (mx > 0.0f && isfinite(mx)) {
        frexpf(mx, &ex);
        ex -= 1;  // mx in [2^ex, 2^(ex+1))
      }
      e_row = static_cast<float>(ex);
    }
    kscale[quad] = F * p.scale_log2 * exp2f(e_row);
    // A operand: lane row (h', g') = (li/4, li%4), non-zero when g' == lane group
    const int ha = quad * 4 + (li >> 2);
    const int ha_c = ha < gqw ? ha : gqw - 1;  // in-range head for unused rows
    const float e_a = __shfl(e_row, (li >> 2) << 4, kWave);
    const bool live = (li & 3) == lq && ha < gqw;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      _Float16 hi[8], lo[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float raw = query_at<QT>(p, head0 + ha_c, qk_dim<BITS>(m, lq, s));
        float x = live ? raw : 0.0f;
        if (kNormalise) x = ldexpf(x, -static_cast<int>(e_a));
        hi[s] = static_cast<_Float16>(x);
        lo[s] = static_cast<_Float16>(x - static_cast<float>(hi[s]));
      }
      qa[quad][0][m] = u32x4{pack_half2(hi[0], hi[1]), pack_half2(hi[2], hi[3]), pack_half2(hi[4], hi[5]),
                             pack_half2(hi[6], hi[7])};
      if (QSPLIT == 2)
        qa[quad][QSPLIT - 1][m] = u32x4{pack_half2(lo[0], lo[1]), pack_half2(lo[2], lo[3]), pack_half2(lo[4], lo[5]),
                                        pack_half2(lo[6], lo[7])};
    }
    // correction -OFF * sum_{d in g} (hi + lo) for head hrow, all 4 groups:
    // lane (row lq, li) sums dims 8li..8li+7 (group li/4); quads of lanes meet
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = query_at<QT>(p, head0 + hrow_c, 8 * li + i);
      if (kNormalise) x = ldexpf(x, -static_cast<int>(e_row));
      const _Float16 h16 = static_cast<_Float16>(x);
      const float rep = QSPLIT == 2 ? static_cast<float>(h16) +
                                          static_cast<float>(static_cast<_Float16>(x - static_cast<float>(h16)))
                                    : static_cast<float>(h16);
      part += rep;
    }
    part += __shfl_xor(part, 1, kWave);
    part += __shfl_xor(part, 2, kWave);
#pragma unroll
    for (int g = 0; g < 4; ++g) qcorr[quad][g] = -OFF * __shfl(part, (lq << 4) + 4 * g, kWave);
  }

  QuadState qs[QUADS];
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    qs[quad].m_run = -INFINITY;
    qs[quad].l_run = 0.0f;
    qs[quad].wsum = 0.0f;
#pragma unroll
    for (int n = 0; n < 8; ++n) qs[quad].acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // ------------------------------------------- software-pipelined main loop
  // stage s0 computes while stage s1's loads are in flight, then swap
  while (have0) {
    const bool have1 = next_sub(cur, p, u_end);
    const Cursor c1 = cur;
    if (have1) issue_loads<BITS>(s1, p, c1, kvh, li, lq);
    process<BITS, QUADS, QSPLIT>(s0, c0, v_lds, w_lds, qa, qcorr, kscale, qs, li, lq);
    if (!have1) break;
    have0 = next_sub(cur, p, u_end);
    c0 = cur;
    if (have0) issue_loads<BITS>(s0, p, c0, kvh, li, lq);
    process<BITS, QUADS, QSPLIT>(s1, c1, v_lds, w_lds, qa, qcorr, kscale, qs, li, lq);
  }

  // ----------------------------------------------------------------- epilogue
  const long prow = static_cast<long>(split) * p.query_heads + head0;
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    const float l_tot = row_sum16(qs[quad].l_run);
    float wtot = qs[quad].wsum;
    wtot += __shfl_xor(wtot, 16, kWave);
    wtot += __shfl_xor(wtot, 32, kWave);
    const int hrow = quad * 4 + lq;
    if (li == 0 && hrow < gqw) {
      p.part_ml[2 * (prow + hrow)] = qs[quad].m_run;
      p.part_ml[2 * (prow + hrow) + 1] = l_tot;
    }
    const int hcol = quad * 4 + (li >> 2);
    const int g = li & 3;
    if (hcol < gqw) {
      float* orow = p.part_o + (prow + hcol) * 128;
      // out = F * (C - OFF * sum W) on the tiles whose dims lie in group g;
      // compile-time tile indices keep the accumulators in registers
      if (BITS == 4) {
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          if ((n >> 1) == g) {
            f32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = F * (qs[quad].acc[n][i] - OFF * wtot);
            *reinterpret_cast<f32x4*>(orow + 16 * n + 4 * lq) = o;
          }
        }
      } else {
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          if (gg == g) {
            const f32x4 ev = qs[quad].acc[2 * gg], od = qs[quad].acc[2 * gg + 1];
            f32x4 o0, o1;
            o0[0] = F * (ev[0] - OFF * wtot);
            o0[1] = F * (od[0] - OFF * wtot);
            o0[2] = F * (ev[1] - OFF * wtot);
            o0[3] = F * (od[1] - OFF * wtot);
            o1[0] = F * (ev[2] - OFF * wtot);
            o1[1] = F * (od[2] - OFF * wtot);
            o1[2] = F * (ev[3] - OFF * wtot);
            o1[3] = F * (od[3] - OFF * wtot);
            *reinterpret_cast<f32x4*>(orow + 32 * gg + 8 * lq) = o0;
            *reinterpret_cast<f32x4*>(orow + 32 * gg + 8 * lq + 4) = o1;
          }
        }
      }
    }
  }
}

template <int BITS, int QUADS, int QSPLIT, typename QT>
void launch_one(const MfmaParams& prm, int grid, bool quad_per_group, hipStream_t s) {
  const DecodeTail rest{prm.valid,       prm.table,      prm.part_o,     prm.part_ml,
                        prm.query_heads, prm.num_blocks, prm.scale_log2, prm.splits};
  hipLaunchKernelGGL((decode_mfma_kernel<BITS, QUADS, QSPLIT, QT>), dim3(grid), dim3(64), 0, s, prm.query, prm.pk,
                     prm.pv, prm.sk, prm.sv, pack_heads(prm.kv_heads, prm.gq, prm.table != nullptr, quad_per_group),
                     prm.block_tokens, prm.blocks_per_split, prm.units, rest);
}

template <int BITS, int QUADS>
int launch_quads(const MfmaParams& prm, int grid, bool quad_per_group, int dtype, hipStream_t s) {
  switch (dtype) {
    case KVSSD_DTYPE_F16:
      launch_one<BITS, QUADS, 1, _Float16>(prm, grid, quad_per_group, s);
      break;
    case KVSSD_DTYPE_BF16:  // 8 significant bits: one fp16 part holds a normalised value exactly
      launch_one<BITS, QUADS, 1, uint16_t>(prm, grid, quad_per_group, s);
      break;
    case KVSSD_DTYPE_F32:
      launch_one<BITS, QUADS, 2, float>(prm, grid, quad_per_group, s);
      break;
    case KVSSD_DTYPE_F64:
      launch_one<BITS, QUADS, 2, double>(prm, grid, quad_per_group, s);
      break;
    default:
      return arg_error("unsupported query dtype");
  }
  return hip_status(hipGetLastError(), "decode_mfma launch");
}

}  // namespace

bool mfma_supported(const kvssd_decode_desc& d, std::string* why) {
  auto no = [&](const char* r) {
    if (why) *why = r;
    return false;
  };
  if (d.head_dim != 128) return no("head_dim must be 128");
  if (d.group_size != 32) return no("group_size must be 32");
  if (d.block_tokens % kSub) return no("block_tokens must be a multiple of 128");
  if (d.kv_heads > 0xFFFF) return no("kv_heads must be below 65536");
  const int gq = d.query_heads / d.kv_heads;
  if (gq < 1 || gq > 8) return no("at most 8 query heads per kv head");
  return true;
}

bool mfma_aligned(const DecodeArgs& a) {
  const uintptr_t need = a.desc.bits == 4 ? 16 : 8;
  auto ok = [&](const void* ptr, uintptr_t al) { return (reinterpret_cast<uintptr_t>(ptr) % al) == 0; };
  return ok(a.packed_k, need) && ok(a.packed_v, need) && ok(a.scales_k, 8) && ok(a.scales_v, 8);
}

int launch_mfma(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts) {
  const kvssd_decode_desc& d = a.desc;
  MfmaParams prm{};
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
  prm.block_tokens = d.block_tokens;
  prm.num_blocks = d.num_blocks;
  prm.units = a.units;
  prm.splits = plan.splits;
  prm.blocks_per_split = plan.blocks_per_split;
  prm.gq = d.query_heads / d.kv_heads;
  prm.scale_log2 = static_cast<float>(d.sm_scale) * kLog2e;
  // More than 4 query heads per kv head: a workgroup per query quad (the
  // one-quad code, half the math per wave) while the doubled grid still fits
  // the GPU's SIMDs at one wave each, so every workgroup starts at once and the
  // codes read twice come from L2 or cost no time on a latency-bound decode;
  // beyond that one workgroup carries both quads and reads the codes once.
  const bool two = prm.gq > 4;
  const bool quad_per_group = two && 2L * plan.splits * d.kv_heads <= kMfmaResidentWaves;
  // ids cover 8 XCD lanes x workgroups per split x ceil(splits / 8); surplus ids exit at once
  const int grid = 8 * d.kv_heads * (quad_per_group ? 2 : 1) * ((plan.splits + 7) / 8);
  if (d.bits == 4) return two && !quad_per_group ? launch_quads<4, 2>(prm, grid, false, d.query_dtype, a.stream)
                                                 : launch_quads<4, 1>(prm, grid, quad_per_group, d.query_dtype, a.stream);
  return two && !quad_per_group ? launch_quads<2, 2>(prm, grid, false, d.query_dtype, a.stream)
                                : launch_quads<2, 1>(prm, grid, quad_per_group, d.query_dtype, a.stream);
}

}  // namespace kvssd
