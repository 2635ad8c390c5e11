// LDS-staged matrix-core decode kernel for gfx950: head_dim 128, group_size 32,
// INT4 or INT2 codes, kv_heads % 4 == 0, at most 8 query heads per kv head,
// block_tokens % 128 == 0.
//
// Same semantics as the general kernel (ReferenceAttentionBackend.run,
// src/kvssd/backends/reference.py:22-50; element addressing of
// csrc/fused_decode.cu:50-56).
//
// Work split.  A workgroup of 8 waves owns KG consecutive kv heads (a
// "group": 4, or 8 when kv_heads % 8 == 0 and the context is long enough to
// fill the chip) and one split (its share of the attended blocks: every
// splits-th one for INT4, a contiguous run for INT2).  It walks the
// split in stages of 512 / KG tokens (128 or 64); wave (w, half) computes kv
// head w of the group over tokens 64*half .. 64*half+63 of every stage.  With
// KG = 4 the two halves meet in LDS at the end; with KG = 8 there is one half.
// Each workgroup writes one partial per query head of its group.  Whole
// 512-byte token rows per workgroup (KG = 8, INT4, 8 kv heads) keep every
// workgroup's copies spread evenly over the memory channels.
//
// Staging.  The packed rows of the group's kv heads of one token are
// contiguous in HBM ([blocks][tokens][kv_heads][packed]), so a stage is four
// contiguous streams (K codes, V codes, K scales, V scales).  They are copied
// HBM -> LDS with global_load_lds_dwordx4 (16 bytes per lane, 1 KB per
// instruction, no VGPRs held while in flight), double-buffered: stage i+1's
// copies are issued right after the barrier that opens stage i, so they
// overlap all of stage i's math.  LDS per stage: 72 KB (INT4) / 40 KB (INT2),
// i.e. 144 KB / 80 KB in total, whatever KG.
//
// LDS layout.  A region stores, per token t of the stage, CPT 16-byte chunks
// (CPT = KG kv heads x packed bytes / 16); chunk idx of token t sits at
// position t*CPT + (idx ^ phi(t)).  phi is chosen so that the matrix-core
// operand reads below hit 16 distinct bank groups per 16 lanes; the DMA lane
// -> global address map applies the inverse, so each copy instruction still
// reads whole 128-byte lines of one contiguous HBM range.
//
// Code -> fp16 without a dequantised tensor: a code c in the mantissa of an
// fp16 whose exponent is that of 1.0 reads as v = 1 + c/F, and
// (c - mid) = F (v - OFF) with OFF = 1 + mid/F (F = 1024 or 64 per slot for
// INT4, 64, 16 or 4 for INT2; absorbed by the query operand in QK and by W or
// the output factor in PV).  The offset is removed through the accumulator: QK starts from
// -sum q' OFF, PV subtracts an extra MFMA of W against OFF (for INT2 both
// parities' OFF in one operand, one per column half).
//
// QK (v_mfma_f32_16x16x32_f16): A = query, rows (h, g) = 4 heads x 4 groups,
//   row (h, g) holding head h masked to group g; B = K codes of a 16-token
//   tile.  Lane (li, lq) ends with the 4 group partials of head lq, token li,
//   and forms s = sum_g scale_k[t, g] * C[g] with fp16-operand FMAs.
// softmax: per-stage max by 16-lane DPP reduction, running (m, l) in log2
//   units, p = 2^(s - m).  W[t, (h, g)] = p * scale_v[t, g] in fp16,
//   written to LDS; m includes a per-stage power of two e set by the stage's
//   largest V scale, which keeps W in fp16's normal range (common.hpp).
// PV (v_mfma_f32_16x16x32_f16): A = W^T, rows (h, g); B = V codes from a
//   16x16 nibble transpose read (ds_read_b64_tr_b4) of the staged V rows, one
//   column per dim: one transpose read covers all 64 tokens of a wave's half
//   for 16 dims (INT4) / 32 dims (INT2).  Lane (li, lq) ends with rows
//   (head lq, groups 0..3) of its dim, of which it keeps the group that owns
//   the dim -- the same head as its scores, so the softmax rescale needs no
//   exchange between lanes and touches only the kept entries.
// Token <-> MFMA K slot (PV, shared by A and B): K step kk, lane group q,
//   slot s -> token 16*(s&3) + 4q + 2kk + (s>>2) of the half; QK tile tau,
//   lane li -> token 16*tau + li.  W of QK lane li, tile tau lives in slot
//   4*u + tau of its (h, g) row, u = 8((li>>1)&1) + 2(li>>2) + (li&1).
#include <type_traits>

#include "staged_ops.hpp"
#include "timeline.hpp"

#ifdef KVSSD_TIMELINE
__device__ uint64_t kvssd_timeline_stamps[kvssd::kTimelineWgs * kvssd::kTimelineSlots];
#endif

namespace kvssd {
namespace {

constexpr int kWaves = 8;            // (kv head, token half)
constexpr int kThreads = 64 * kWaves;
constexpr int kHalfTok = 64;         // tokens per wave per stage
constexpr int kMaxUnits = 2048;      // attended blocks per split (block list kept in LDS)
template <int KG>
constexpr int kStageTok = kWaves / KG * kHalfTok;  // tokens per stage: 128 (KG 4) or 64 (KG 8)

template <int BITS, int KG>
struct Geo {
  static constexpr int PD = 128 * BITS / 8;               // packed bytes per kv-head row
  static constexpr int CPT = KG * PD / 16;                // chunks per token row of the group
  static constexpr int SCPT = KG * 8 / 16;                // chunks per scale row of the group
  static constexpr int HALVES = kWaves / KG;
  static constexpr int KV_BYTES = kStageTok<KG> * KG * PD;  // one code region
  static constexpr int SC_BYTES = kStageTok<KG> * KG * 8;   // one scale region
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = KV_BYTES;
  static constexpr int SK_OFF = 2 * KV_BYTES;
  static constexpr int SV_OFF = 2 * KV_BYTES + SC_BYTES;
  static constexpr int STAGE = 2 * KV_BYTES + 2 * SC_BYTES;
  static constexpr int KV_INST = KV_BYTES / 1024;         // copy instructions per code region
  static constexpr int SC_INST = SC_BYTES / 1024;         // ... per scale region
  static constexpr int KV_PER_WAVE = KV_INST / kWaves;
  // INT4: W lives in the wave's own (already consumed) K chunks of the stage;
  // INT2 K chunks are too few for two query quads, so W gets its own region.
  static constexpr bool W_IN_K = BITS == 4;
};
static_assert(Geo<4, 4>::SC_INST * 2 == kWaves && Geo<2, 4>::SC_INST * 2 == kWaves && Geo<4, 8>::SC_INST * 2 == kWaves &&
                  Geo<2, 8>::SC_INST * 2 == kWaves,
              "one scale copy per wave");

struct StagedParams {
  const void* query;
  const uint8_t* pk;
  const uint8_t* pv;
  const uint8_t* sk;  // fp16 scales as bytes
  const uint8_t* sv;
  const int32_t* valid;
  const int32_t* table;
  float* part_o;
  float* part_ml;
  int query_heads, kv_heads, block_tokens, num_blocks, units;
  int split_arg;  // the number of splits (interleaved split order) or blocks per split (contiguous)
  int gq;
  float scale_log2;  // sm_scale * log2(e)
};

// Which units a split attends.  Interleaved: split s takes units s, s + splits,
// s + 2 splits, ..., so at any moment the workgroups stream neighbouring
// blocks.  With a contiguous run of blocks per split their streams sit a fixed
// power-of-two distance apart (256 KB of K codes at 128K), and HBM serves that
// pattern slower: a plain read of the INT4 128K layer in this kernel's stage
// pattern (256 workgroups, 64-token stages of K, V and scales, plain loads)
// took 29.1 us that way against 25.7 us interleaved, and the INT4 128K split
// kernel went 28.5-28.8 -> 27.0-27.2 us (A/B pairs; 1M 0.2-1.5 us faster).
// INT2's stage round is bound by its math, not by its reads; it measured
// 0.1 us slower interleaved (128K) and keeps the contiguous runs.
template <int BITS>
constexpr bool kInterleavedSplits = BITS == 4;

// XOR swizzle of a region's chunk index for token t (CPT chunks per token).
// A token row of 16 or more chunks spans every bank group, so the swizzle
// only permutes its low 4 bits (the same for CPT 16 and 32).
template <int CPT>
__device__ __forceinline__ int phi(int t) {
  if constexpr (CPT >= 16) return (t & 15) ^ (((t >> 4) & 3) << 2);
  else if constexpr (CPT == 8) return ((t & 15) >> 1) ^ (((t >> 4) & 3) << 1);
  else if constexpr (CPT == 4) return (t >> 2) & 3;  // scale rows of 8 kv heads
  else return (t >> 3) & 1;                          // CPT == 2: scale rows of 4 kv heads
}

template <int CPT>
__device__ __forceinline__ int chunk_byte(int t, int idx) {
  return 16 * (t * CPT + (idx ^ phi<CPT>(t)));
}

// Per-lane byte offsets (relative to the stage's group base) of this wave's
// copy instructions.  Copy j of a code region (lane positions 64 (wave + 8 j)
// + lane) covers token row t0 + j * 512 / CPT, with copy 0's slot: its
// swizzle differs from copy 0's by phi(j * 512 / CPT) whatever t0 (the row's
// bits 4 and up reach phi only as an XOR of chunk bits, and t0's low bits are
// the same for every j), so two registers serve every copy: the row offset
// and the swizzled chunk offset, XORed with a constant per copy; the row step
// goes into the scalar base.  One more register holds the scale copy's offset.
template <int BITS, int KG>
struct CopyMap {
  uint32_t row;    // t0 * row stride
  uint32_t chunk;  // 16 * (slot ^ phi(t0))
  uint32_t sc;
};

template <int BITS, int KG>
__device__ __forceinline__ CopyMap<BITS, KG> make_copy_map(int wave, int lane, int kv_heads) {
  using G = Geo<BITS, KG>;
  CopyMap<BITS, KG> cm;
  const int pos0 = 64 * wave + lane;
  const int t0 = pos0 / G::CPT, slot0 = pos0 % G::CPT;
  cm.row = static_cast<uint32_t>(t0 * kv_heads * G::PD);
  cm.chunk = static_cast<uint32_t>(16 * (slot0 ^ phi<G::CPT>(t0)));
  const int pos = 64 * (wave & 3) + lane;
  const int t = pos / G::SCPT, slot = pos % G::SCPT;
  cm.sc = static_cast<uint32_t>(t * kv_heads * 8 + 16 * (slot ^ phi<G::SCPT>(t)));
  return cm;
}

template <int BITS, int KG>
__device__ __forceinline__ void issue_stage(const StagedParams& p, uint32_t buf, const Cursor& c, int kvh0, int wave,
                                            const CopyMap<BITS, KG>& cm) {
  using G = Geo<BITS, KG>;
  constexpr int kRowStep = kThreads / G::CPT;  // token rows between a wave's copies
  const long row0 = (static_cast<long>(c.blk) * p.block_tokens + c.sb0) * p.kv_heads + kvh0;
  // the scale copy first: should its offset ever be reloaded from scratch, the
  // wait for it does not also wait for this stage's code copies
  const uint8_t* sb = (wave < 4 ? p.sk : p.sv) + row0 * 8;
  dma16<false>(sb, cm.sc, buf + (wave < 4 ? G::SK_OFF : G::SV_OFF) + 1024u * static_cast<uint32_t>(wave & 3));
  const long rs = static_cast<long>(p.kv_heads) * G::PD;
#pragma unroll
  for (int j = 0; j < G::KV_PER_WAVE; ++j) {
    const uint32_t i = static_cast<uint32_t>(wave + kWaves * j);
    const uint32_t off = (cm.chunk ^ static_cast<uint32_t>(16 * phi<G::CPT>(j * kRowStep))) + cm.row;
    const long step = static_cast<long>(j) * kRowStep * rs;
    dma16<true>(p.pk + row0 * G::PD + step, off, buf + G::K_OFF + 1024u * i);
    dma16<true>(p.pv + row0 * G::PD + step, off, buf + G::V_OFF + 1024u * i);
  }
}

// W chunk (quad, row R = 4h + g, chunk c of 8 slots) byte offset.
template <int BITS, int QUADS, int KG>
__device__ __forceinline__ int w_chunk(int quad, int R, int c, int w, int half) {
  using G = Geo<BITS, KG>;
  if constexpr (G::W_IN_K) {
    // inside the wave's K chunks (kv head w, tokens of its half) of the stage
    const int b = c >> 2;
    const int t = kHalfTok * half + 32 * quad + (R & 7) + 8 * ((R >> 3) ^ b) + 16 * b;
    return G::K_OFF + chunk_byte<G::CPT>(t, 4 * w + (c & 3));
  } else {
    // own region after both stage buffers, [wave][quad][row][8 chunks]
    const int rp = R ^ ((R >> 2) & 1);
    return quad * 2048 + rp * 128 + 16 * (c ^ ((rp >> 1) & 7));
  }
}

// ---------------------------------------------------------- per-wave state ---
template <int BITS, int QUADS>
struct WaveState {
  float m_run[QUADS], l_run[QUADS];
  f32x4 acc[QUADS][8];
  // sum over tokens of W * OFF, rows (head, group); INT2 keeps parity 0's OFF
  // in columns (lanes li) 0-7 and parity 1's in 8-15 of one accumulator
  f32x4 corr[QUADS];
};

// One stage of one wave: tokens 64*half .. 64*half + hv - 1 of the stage are valid.
// Every LDS read of the stage goes out first, the four tiles' QK chains are
// interleaved and V is unpacked before the softmax, so the two waves of a
// SIMD have independent work to fill each other's latencies.
template <int BITS, int QUADS, int QSPLIT, int KG>
__device__ __forceinline__ void compute_stage(const uint8_t* buf, uint8_t* wbase, int hv, int w, int half, int li,
                                              int lq, const Masks& mk, const QueryOps<QUADS, QSPLIT>& qo,
                                              const u32x4& offa, WaveState<BITS, QUADS>& st) {
  using G = Geo<BITS, KG>;
  constexpr int KW = BITS == 4 ? 4 : 2;   // K words per lane and tile
  constexpr int NTR = BITS == 4 ? 8 : 4;  // transpose reads (16 / 32 dims each)
  constexpr int NPAR = BITS == 4 ? 1 : 2;
  // ------------------------------------------------------------ LDS reads
  uint32_t kraw[4][KW];
  u32x2 skw[4], svw[4];
#pragma unroll
  for (int tau = 0; tau < 4; ++tau) {
    const int t = kHalfTok * half + 16 * tau + li;
    if (BITS == 4) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(buf + G::K_OFF + chunk_byte<G::CPT>(t, 4 * w + lq));
#pragma unroll
      for (int i = 0; i < KW; ++i) kraw[tau][i] = r[i];
    } else {
      const u32x2 r =
          *reinterpret_cast<const u32x2*>(buf + G::K_OFF + chunk_byte<G::CPT>(t, 2 * w + (lq >> 1)) + 8 * (lq & 1));
#pragma unroll
      for (int i = 0; i < KW; ++i) kraw[tau][i] = r[i];
    }
    const int sbyte = chunk_byte<G::SCPT>(t, w >> 1) + 8 * (w & 1);
    skw[tau] = *reinterpret_cast<const u32x2*>(buf + G::SK_OFF + sbyte);
    svw[tau] = *reinterpret_cast<const u32x2*>(buf + G::SV_OFF + sbyte);
  }
  // the V scales of tile lq's token li: the lanes of the wave hold the
  // stage's 64 tokens once each (for the stage's scale exponent)
  u32x2 svm = *reinterpret_cast<const u32x2*>(
      buf + G::SV_OFF + chunk_byte<G::SCPT>(kHalfTok * half + 16 * lq + li, w >> 1) + 8 * (w & 1));
  // transpose-read row of this lane: kk = li >> 3, row rho = li & 7,
  // slot s = 2(rho & 3) + (rho >> 2) -> token 16(s&3) + 4lq + 2kk + (s>>2)
  const int rho = li & 7;
  const int s_tr = ((rho & 3) << 1) | (rho >> 2);
  const int t_tr = kHalfTok * half + 16 * (s_tr & 3) + 4 * lq + 2 * (li >> 3) + (s_tr >> 2);
  // (two query quads keep twice the accumulators live: their V reads and
  // unpack wait until after the softmax so the operands fit the registers)
  constexpr bool kEarlyV = QUADS == 1;
  i32x2 tr[NTR];
  auto read_v = [&]() {
#pragma unroll
    for (int n = 0; n < NTR; ++n)
      tr[n] = BITS == 4 ? lds_read_tr4(buf, G::V_OFF + chunk_byte<G::CPT>(t_tr, 4 * w + (n >> 1)) + 8 * (n & 1))
                        : lds_read_tr4(buf, G::V_OFF + chunk_byte<G::CPT>(t_tr, 2 * w + (n >> 1)) + 8 * (n & 1));
  };
  if constexpr (kEarlyV) {
    read_v();
    // (keeps the transpose reads here, with the stage's other LDS reads: the
    // scheduler would otherwise move them after the QK math, and the PV then
    // waits out their latency)
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---------------------------------------------------------------- QK
  f32x4 cc[QUADS][4];
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) cc[quad][tau] = qo.qcorr[quad];
  if constexpr (kEarlyV) {
    // the four tiles' chains interleaved, one K word position at a time
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      u32x4 b[4];
#pragma unroll
      for (int tau = 0; tau < 4; ++tau)
        b[tau] = BITS == 4 ? unpack4(kraw[tau][m], mk) : unpack2(kraw[tau][m >> 1], m & 1, mk);
#pragma unroll
      for (int sp = 0; sp < QSPLIT; ++sp)
#pragma unroll
        for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
          for (int tau = 0; tau < 4; ++tau) cc[quad][tau] = mfma16(qo.qa[quad][sp][m], b[tau], cc[quad][tau]);
    }
  } else {
    // tile by tile (fewer live operands)
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
      u32x4 b[4];
#pragma unroll
      for (int m = 0; m < 4; ++m)
        b[m] = BITS == 4 ? unpack4(kraw[tau][m], mk) : unpack2(kraw[tau][m >> 1], m & 1, mk);
#pragma unroll
      for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
        for (int sp = 0; sp < QSPLIT; ++sp)
#pragma unroll
          for (int m = 0; m < 4; ++m) cc[quad][tau] = mfma16(qo.qa[quad][sp][m], b[m], cc[quad][tau]);
    }
  }
  float score[QUADS][4];
#pragma unroll
  for (int tau = 0; tau < 4; ++tau) {
#pragma unroll
    for (int quad = 0; quad < QUADS; ++quad) {
      const f32x4 c = cc[quad][tau];
      float raw = __builtin_fmaf(half_lo(skw[tau][0]), c[0], 0.0f);
      raw = __builtin_fmaf(half_hi(skw[tau][0]), c[1], raw);
      raw = __builtin_fmaf(half_lo(skw[tau][1]), c[2], raw);
      raw = __builtin_fmaf(half_hi(skw[tau][1]), c[3], raw);
      score[quad][tau] = raw * qo.kscale[quad];
    }
  }
  // a partial stage (uniform branch): tokens past the valid count get score
  // -inf and value scale 0 (p is 0 there, but the stale scale may not be finite)
  if (hv < kHalfTok) {
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
      if (16 * tau + li >= hv) {
#pragma unroll
        for (int quad = 0; quad < QUADS; ++quad) score[quad][tau] = -INFINITY;
        svw[tau] = u32x2{0u, 0u};
      }
    }
    if (16 * lq + li >= hv) svm = u32x2{0u, 0u};
  }
  // the stage's V-scale exponent (wave-uniform): W = 2^(s - (m + e)) scale_v
  // stays in fp16's normal range, whatever the range of the scales
  const float e_v = static_cast<float>(wave_scale_exp(abs_max_bits(svm[0], svm[1])));
  // --------------------------------------------- V operands (no softmax dep)
  u32x4 va[NTR][2][NPAR];
  auto unpack_v = [&]() {
#pragma unroll
    for (int n = 0; n < NTR; ++n)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int par = 0; par < NPAR; ++par)
          va[n][kk][par] = BITS == 4 ? unpack4(static_cast<uint32_t>(tr[n][kk]), mk)
                                     : unpack2_tr(static_cast<uint32_t>(tr[n][kk]), par, mk);
  };
  if constexpr (kEarlyV) unpack_v();
  // unit of this lane's W slots (4 tiles) in its (h, g) rows
  const int u = 8 * ((li >> 1) & 1) + 2 * (li >> 2) + (li & 1);
  // --------------------------------------------------------------- softmax
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    // (the running reference is max over stages of the stage max plus e)
    const float mx = row_max16_of(score[quad][0], score[quad][1], score[quad][2], score[quad][3]) + e_v;
    const float m_new = fmaxf(st.m_run[quad], mx);
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(st.m_run[quad] - m_new);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    st.m_run[quad] = m_new;
    float pr[4];
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) pr[tau] = __builtin_amdgcn_exp2f(score[quad][tau] - m_use);
    st.l_run[quad] = st.l_run[quad] * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    // W = p * scale_v in fp16 (masked tokens: p = 0, scale 0), p relative to
    // m + e so that W <= 2^11; INT4 tiles 0, 1 sit in the K slots with
    // F = 1024, so their W carries F/64 = 16 (at most 2^15).
    // Each fp16 pair is one mixed-precision FMA into each half.
    uint32_t wlo[4], whi[4];  // per group g: (tile 0, tile 1), (tile 2, tile 3)
#pragma unroll
    for (int tau = 0; tau < 4; tau += 2) {
      const float wfac = (BITS == 4 && tau == 0) ? 16.0f : 1.0f;
      const float p0 = pr[tau] * wfac, p1 = pr[tau + 1] * wfac;
      const uint32_t a01 = svw[tau][0], a23 = svw[tau][1];
      const uint32_t b01 = svw[tau + 1][0], b23 = svw[tau + 1][1];
      const uint32_t w0 = wpair(p0, half_lo(a01), p1, half_lo(b01));
      const uint32_t w1 = wpair(p0, half_hi(a01), p1, half_hi(b01));
      const uint32_t w2 = wpair(p0, half_lo(a23), p1, half_lo(b23));
      const uint32_t w3 = wpair(p0, half_hi(a23), p1, half_hi(b23));
      if (tau == 0) {
        wlo[0] = w0; wlo[1] = w1; wlo[2] = w2; wlo[3] = w3;
      } else {
        whi[0] = w0; whi[1] = w1; whi[2] = w2; whi[3] = w3;
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int off = w_chunk<BITS, QUADS, KG>(quad, 4 * lq + g, u >> 1, w, half) + 8 * (u & 1);
      *reinterpret_cast<u32x2*>(wbase + off) = u32x2{wlo[g], whi[g]};
    }
    // rescale the PV state of head lq (the same head as this lane's scores):
    // only the entries the epilogue reads, group k/2 of tile k
#pragma unroll
    for (int k = 0; k < 8; ++k) st.acc[quad][k][k >> 1] *= alpha;
#pragma unroll
    for (int g = 0; g < 4; ++g) st.corr[quad][g] *= alpha;
  }
  // -------------------------------------------------------------------- PV
  if constexpr (!kEarlyV) {
    read_v();
    unpack_v();
  }
  u32x4 wb[QUADS][2];
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      wb[quad][kk] = *reinterpret_cast<const u32x4*>(wbase + w_chunk<BITS, QUADS, KG>(quad, li, 4 * kk + lq, w, half));
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int n = 0; n < NTR; ++n)
#pragma unroll
      for (int par = 0; par < NPAR; ++par)
#pragma unroll
        for (int quad = 0; quad < QUADS; ++quad)
          st.acc[quad][NPAR * n + par] = mfma16(wb[quad][kk], va[n][kk][par], st.acc[quad][NPAR * n + par]);
  // sum over tokens of W * OFF per row, through the matrix core
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) st.corr[quad] = mfma16(wb[quad][kk], offa, st.corr[quad]);
}

// s_waitcnt vmcnt(BASE + extra), extra in [0, 4] and wave-uniform (a
// larger value, which the host's kMaxUnits check rules out, waits for BASE)
template <int BASE>
__device__ __forceinline__ void wait_copies_left(int extra) {
  switch (extra) {
    case 1: __builtin_amdgcn_s_waitcnt(vmcnt_wait(BASE + 1)); break;
    case 2: __builtin_amdgcn_s_waitcnt(vmcnt_wait(BASE + 2)); break;
    case 3: __builtin_amdgcn_s_waitcnt(vmcnt_wait(BASE + 3)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_wait(BASE + 4)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_wait(BASE)); break;
  }
}

// INT2's stage round is bound by its VALU: with the stage loop unrolled by the
// two stage buffers, every LDS address of a stage is a loop-invariant lane
// offset plus a constant the LDS instructions take as their immediate offset
// (a runtime buffer costs ~10 address adds per wave and stage): the INT2 128K
// GQA-4 step 23.5-23.6 -> 23.25-23.3 us (two rounds of three A/B pairs, one
// box each), GQA 8 unchanged.  INT4 measured no faster with it (128K within
// +-0.15 us, 256K and 1M within 1 us either way, A/B pairs) and keeps the loop
// below; the two-quad fp32 / fp64 INT2 form would spill.
template <int BITS, int QUADS, int QSPLIT>
constexpr bool kUnrollByBuffer = BITS == 2 && !(QUADS == 2 && QSPLIT == 2);

template <int BITS, int QUADS, int QSPLIT, typename QT, int KG>
__global__ __launch_bounds__(kThreads) void decode_staged_kernel(const void* query, const uint8_t* pk,
                                                                 const uint8_t* pv, const uint8_t* sk,
                                                                 const uint8_t* sv, uint32_t heads, int block_tokens,
                                                                 int split_arg, int units_total, DecodeTail r) {
  const StagedParams p{query,           pk,
                       pv,              sk,
                       sv,              r.valid,
                       r.table,         r.part_o,
                       r.part_ml,       r.query_heads,
                       static_cast<int>(heads & 0xFFFFu), block_tokens,
                       r.num_blocks,    units_total,
                       split_arg,       static_cast<int>((heads >> 16) & 0xFFu),
                       r.scale_log2};
  const bool has_table = (heads & kHasTable) != 0;
  // the non-preloaded arguments, in SGPRs from here on (they stay live, so no
  // register of theirs is reused before this point)
  auto rest_in_sgprs = [&] {
    asm volatile("" ::"s"(r.valid), "s"(r.table), "s"(r.part_o), "s"(r.part_ml), "s"(r.query_heads),
                 "s"(r.num_blocks), "s"(r.scale_log2), "s"(r.splits));
  };
  using G = Geo<BITS, KG>;
  constexpr int kStage = kStageTok<KG>;
  constexpr int kWBytes = G::W_IN_K ? 0 : kWaves * QUADS * 2048;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * G::STAGE + kWBytes + kMaxUnits * 8];

  KVSSD_STAMP(kStampEntry);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int w = wave & (KG - 1);
  const int half = wave / KG;
  const int li = lane & 15;
  const int lq = lane >> 4;

  // workgroup -> (split, group of KG kv heads).  Consecutive workgroup ids go
  // to different XCDs (round robin over 8); every group of split s gets an id
  // with id % 8 == s % 8, so they share one XCD and its L2: the groups read
  // complementary parts of the same 128-byte lines of the scale rows.
  const int groups = p.kv_heads / KG;
  const int xcd = blockIdx.x & 7;
  const int rest = blockIdx.x >> 3;
  const int grp = rest % groups;
  const int split = (rest / groups) * 8 + xcd;
  // the split's units: u_first, u_first + u_stride, ... (n_units of them)
  constexpr bool kInterleave = kInterleavedSplits<BITS>;
  const int u_first = kInterleave ? split : split * p.split_arg;
  const int u_stride = kInterleave ? p.split_arg : 1;
  // padding ids of the last round (splits = ceil(units / blocks per split))
  if (kInterleave ? split >= p.split_arg : u_first >= p.units) return;
  const int u_end = kInterleave ? p.units : min(p.units, u_first + p.split_arg);  // contiguous: the run's end
  const int kvh0 = grp * KG;
  const int head0 = (kvh0 + w) * p.gq;

  const CopyMap<BITS, KG> cm = make_copy_map<BITS, KG>(wave, lane, p.kv_heads);
  const uint32_t lds0 = lds_addr(lds);
  int* units = reinterpret_cast<int*>(lds + 2 * G::STAGE + kWBytes);
  // At least one (splits <= units); at most blocks per split <= kMaxUnits,
  // checked on the host (interleaved: ceil(units / splits) <= blocks per split).
  const int n_units = kInterleave ? (p.units - 1 - split) / u_stride + 1 : max(0, u_end - u_first);

  // Early form (no block table, the query 16-byte aligned, and room in the
  // second stage buffer for the query scratch and the workgroup's query
  // rows): every early memory operation is an LDS copy, so no compiler-placed
  // wait for a load can also wait for a stage.  The query rows go first, then
  // stage 0 and the split's valid counts (one copy per 64 units); once the
  // rows land the query operands are built and stage 1 goes out,
  // before stage 0 has landed: the start is latency-bound, and two stages in
  // flight arrive nearly as soon as one.
  constexpr int kStageCopies = 2 * G::KV_PER_WAVE + 1;    // copy instructions per wave per stage
  constexpr int kQBytesMax = KG * 4 * QUADS * 128 * static_cast<int>(sizeof(QT));
  constexpr bool kEarlyFits = kWaves * coop_scratch_bytes<QUADS> + kQBytesMax <= G::STAGE;
  const bool direct = kEarlyFits && !has_table && (reinterpret_cast<uintptr_t>(p.query) & 15u) == 0;
  auto advance = [&](Cursor& c) -> bool {
    return direct ? next_stage_direct<kStage>(c, units, u_first, u_stride, p.block_tokens, n_units)
                  : next_stage<kStage>(c, units, n_units);
  };

  QueryOps<QUADS, QSPLIT> qo;
  Cursor cur{-1, 0, 0, -kStage};
  Cursor nxt{-1, 0, 0, -kStage};
  bool have = false, have_n = false;
  bool pre1 = false;   // stage 1 went out early and is the loop's second stage
  bool wait0 = true;   // the loop's first pass waits for its stage and meets the barrier
  bool spec = false;   // stage 0 (the split's first block, its first stage of tokens) went out early
  if (direct) {
    uint8_t* qrows = lds + 2 * G::STAGE - kQBytesMax;  // tail of the second stage buffer
    const int qcopies = KG * p.gq * 128 * static_cast<int>(sizeof(QT)) / 1024;
    const uint8_t* qsrc =
        static_cast<const uint8_t*>(p.query) + static_cast<long>(kvh0) * p.gq * 128 * static_cast<long>(sizeof(QT));
    for (int i = wave; i < qcopies; i += kWaves)
      dma16<false>(qsrc, 1024u * static_cast<uint32_t>(i) + 16u * static_cast<uint32_t>(lane),
                   lds_addr(qrows) + 1024u * static_cast<uint32_t>(i));
    if (n_units > 0) {
      issue_stage<BITS, KG>(p, lds0, Cursor{0, u_first, 0, 0}, kvh0, wave, cm);
      spec = true;
    }
    rest_in_sgprs();
    // the split's valid counts, 64 per copy (lanes past the end re-read the
    // last one): the only early copies whose address is not preloaded, so
    // they go last; they are first read once stage 0 has landed
    const uint8_t* vsrc = reinterpret_cast<const uint8_t*>(p.valid + (n_units > 0 ? u_first : 0));
    const int ulast = max(n_units - 1, 0);
    int vcopies = 0;
    for (int i0 = 64 * wave; i0 < n_units; i0 += 64 * kWaves, ++vcopies)
      dma4(vsrc, 4u * static_cast<uint32_t>(min(i0 + lane, ulast) * u_stride),
           lds_addr(reinterpret_cast<const uint8_t*>(units)) + 4u * static_cast<uint32_t>(i0));
    KVSSD_STAMP(kStampStage0Issued);
    // the query rows (issued first) have landed once at most the stage's
    // copies and the valid counts are outstanding (copies complete in issue
    // order)
    if (spec) wait_copies_left<kStageCopies>(vcopies);
    else __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    KVSSD_STAMP(kStampRowsLanded);
    coop_query_build<BITS, QUADS, QSPLIT>(qo, coop_query_load<BITS, QUADS, QT>(qrows, p.gq, w * p.gq, lane),
                                          p.scale_log2, lane, lds + G::STAGE + wave * coop_scratch_bytes<QUADS>);
    __syncthreads();  // query rows and scratch consumed: the second buffer is free
    Cursor c1{-1, 0, 0, 0};
    bool issued1 = false;
    if (spec) {
      if (p.block_tokens > kStage) {
        c1 = Cursor{0, u_first, 0, kStage};
        issued1 = true;
      } else if (n_units > 1) {
        c1 = Cursor{1, u_first + u_stride, 0, 0};
        issued1 = true;
      }
      if (issued1) issue_stage<BITS, KG>(p, lds0 + static_cast<uint32_t>(G::STAGE), c1, kvh0, wave, cm);
    }
    KVSSD_STAMP(kStampStage1Issued);
    // stage 0 and the valid counts landed (only stage 1 may still be in flight)
    if (issued1) __builtin_amdgcn_s_waitcnt(vmcnt_wait(kStageCopies));
    else __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    KVSSD_STAMP(kStampStage0Landed);
    have = advance(cur);
    wait0 = false;
    if (have && !(spec && cur.u == 0 && cur.sb0 == 0)) {
      // the first valid stage is elsewhere (empty or partial blocks): let this
      // wave's early copies land, then load the right ones
      __builtin_amdgcn_s_waitcnt(0x0F70);
      issue_stage<BITS, KG>(p, lds0, cur, kvh0, wave, cm);
      wait0 = true;
    }
    nxt = cur;
    have_n = have && advance(nxt);
    pre1 = issued1 && have_n && nxt.blk == c1.blk && nxt.sb0 == c1.sb0;
    if (issued1 && !pre1) wait0 = true;  // the early stage 1 must land before its buffer is reloaded
  } else {
    // The first stage's copies go out before anything else: the split's first
    // attended block, its first stage of tokens (one scalar read with a block
    // table).  If that block holds no valid token they are simply not used.
    rest_in_sgprs();
    if (n_units > 0) {
      Cursor c0{0, __builtin_amdgcn_readfirstlane(p.table ? p.table[u_first] : u_first), 0, 0};
      if (c0.blk >= 0 && c0.blk < p.num_blocks) {
        issue_stage<BITS, KG>(p, lds0, c0, kvh0, wave, cm);
        spec = true;
      }
    }
    // the query loads go out next: they complete in issue order, right after
    // the first stage's copies, instead of a round trip after them
    const QueryRaw<QUADS> qraw = coop_query_load<BITS, QUADS, QT>(p.query, p.gq, head0, lane);
    // the split's (block id, clamped valid count) list, read once into LDS
    for (int i = threadIdx.x; i < n_units; i += kThreads) {
      const int ui = u_first + i * u_stride;
      const int blk = p.table ? p.table[ui] : ui;
      units[2 * i] = blk;
      units[2 * i + 1] = (blk < 0 || blk >= p.num_blocks) ? 0 : clamp_valid(p.valid[blk], p.block_tokens);
    }
    __syncthreads();
    have = advance(cur);
    if (have && !(spec && cur.u == 0 && cur.sb0 == 0)) {
      __builtin_amdgcn_s_waitcnt(0x0F70);
      issue_stage<BITS, KG>(p, lds0, cur, kvh0, wave, cm);
    }
    // query operands, through per-wave scratch in the second stage buffer (its
    // first copies go out after the loop's first barrier)
    coop_query_build<BITS, QUADS, QSPLIT>(qo, qraw, p.scale_log2, lane,
                                          lds + G::STAGE + wave * coop_scratch_bytes<QUADS>);
    nxt = cur;
    have_n = have && advance(nxt);
  }
  static_assert(kWaves * coop_scratch_bytes<QUADS> <= G::STAGE, "query scratch fits a stage buffer");
  // masks in VGPRs: p.units >= 1, so (lane & (p.units >> 30)) is 0 but opaque
  const Masks mk = make_masks(static_cast<uint32_t>(lane) & static_cast<uint32_t>(p.units >> 30));
  // correction operand: INT4, OFF of each K slot; INT2, a column per lane li:
  // parity 0's OFF (F = 4) in columns 0-7, parity 1's (F = 16) in 8-15
  const u32x4 offa = BITS == 4 ? off_operand4() : off_operand(li < 8 ? 1.5f : 1.125f);

  WaveState<BITS, QUADS> st;
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    st.m_run[quad] = -INFINITY;
    st.l_run[quad] = 0.0f;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.acc[quad][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    st.corr[quad] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // ------------------------------------------- double-buffered stage loop
  // the stage after the current one is looked up a step ahead, so that its
  // copies go out right after the barrier
  bool first = true;
  [[maybe_unused]] int stage_no = 0;
  KVSSD_STAMP(kStampLoop);
  if constexpr (kUnrollByBuffer<BITS, QUADS, QSPLIT>) {
    // one pass with the stage buffer B a compile-time constant
    auto pass = [&](auto buffer) {
      constexpr int B = decltype(buffer)::value;
      if (!first || wait0) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies of the stage landed
        __syncthreads();                     // ... everyone's; and the other buffer is free
      }
      KVSSD_STAMP(kStampStage + min(stage_no++, 15));
      if (have_n && !(first && pre1))
        issue_stage<BITS, KG>(p, lds0 + static_cast<uint32_t>((B ^ 1) * G::STAGE), nxt, kvh0, wave, cm);
      first = false;
      const int hv = min(kStage, cur.vb - cur.sb0) - kHalfTok * half;
      if (hv > 0) {
        uint8_t* sbuf = lds + B * G::STAGE;
        uint8_t* wbase = G::W_IN_K ? sbuf : lds + 2 * G::STAGE + wave * QUADS * 2048;
        compute_stage<BITS, QUADS, QSPLIT, KG>(sbuf, wbase, hv, w, half, li, lq, mk, qo, offa, st);
      }
      cur = nxt;
      have = have_n;
      if (have) have_n = advance(nxt);
    };
    while (have) {
      pass(std::integral_constant<int, 0>{});
      if (!have) break;
      pass(std::integral_constant<int, 1>{});
    }
  } else {
    int buf = 0;
    while (have) {
      if (!first || wait0) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies of the stage landed
        __syncthreads();                     // ... everyone's; and the other buffer is free
      }
      KVSSD_STAMP(kStampStage + min(stage_no++, 15));
      if (have_n && !(first && pre1))
        issue_stage<BITS, KG>(p, lds0 + static_cast<uint32_t>((buf ^ 1) * G::STAGE), nxt, kvh0, wave, cm);
      first = false;
      const int hv = min(kStage, cur.vb - cur.sb0) - kHalfTok * half;
      if (hv > 0) {
        uint8_t* sbuf = lds + buf * G::STAGE;
        uint8_t* wbase = G::W_IN_K ? sbuf : lds + 2 * G::STAGE + wave * QUADS * 2048;
        compute_stage<BITS, QUADS, QSPLIT, KG>(sbuf, wbase, hv, w, half, li, lq, mk, qo, offa, st);
      }
      cur = nxt;
      have = have_n;
      if (have) have_n = advance(nxt);
      buf ^= 1;
    }
  }

  KVSSD_STAMP(kStampLoopEnd);
  // -------------------------------------------------------------- epilogue
  // lane (li, lq) holds head lq of each quad; the entry of tile k it keeps
  // is that of group k/2: dim 16k + li (INT4) or 32(k/2) + 2li + (k & 1)
  // (INT2), and out = F (C - corr) with F = 64 (INT4) or 4 / 16 (INT2
  // parity 0 / 1)
  float* xo = reinterpret_cast<float*>(lds);  // [w][quad][lane][8] from half 1
  float* xm = xo + KG * QUADS * 64 * 8;       // [w][quad][4 heads][2]
  __builtin_amdgcn_s_waitcnt(0x0F70);  // no copy of this wave is still writing LDS
  if constexpr (G::HALVES == 2) __syncthreads();  // every wave is done with the stage buffers
  float ov[QUADS][8];
  float mh[QUADS], lh[QUADS];
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    // INT2: this lane's correction column holds one parity's OFF; the other
    // parity's is in the lane 8 columns away (the same rows: head lq)
    f32x4 corr_par[2];
    if constexpr (BITS == 2) {
      f32x4 other;
#pragma unroll
      for (int g = 0; g < 4; ++g) other[g] = __shfl_xor(st.corr[quad][g], 8, kWave);
      corr_par[0] = li < 8 ? st.corr[quad] : other;
      corr_par[1] = li < 8 ? other : st.corr[quad];
    } else {
      corr_par[0] = corr_par[1] = st.corr[quad];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int g = k >> 1;
      const float f = BITS == 4 ? 64.0f : ((k & 1) ? 16.0f : 4.0f);
      ov[quad][k] = f * (st.acc[quad][k][g] - corr_par[BITS == 4 ? 0 : (k & 1)][g]);
    }
    // (m, l) of head lq: m is the same in the head's 16 lanes, l a per-lane part
    mh[quad] = st.m_run[quad];
    lh[quad] = row_sum16(st.l_run[quad]);
    if (G::HALVES == 2 && half == 1) {
      float* dst = xo + ((w * QUADS + quad) * 64 + lane) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) dst[i] = ov[quad][i];
      if (li == 0) {
        xm[((w * QUADS + quad) * 4 + lq) * 2] = mh[quad];
        xm[((w * QUADS + quad) * 4 + lq) * 2 + 1] = lh[quad];
      }
    }
  }
  if constexpr (G::HALVES == 2) {
    __syncthreads();
    if (half == 1) return;
  }
  const long prow = static_cast<long>(split) * p.query_heads + head0;
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    // the other half's state (none with one half per stage)
    const float* src = xo + ((w * QUADS + quad) * 64 + lane) * 8;
    const float mb = G::HALVES == 2 ? xm[((w * QUADS + quad) * 4 + lq) * 2] : -INFINITY;
    const float lb = G::HALVES == 2 ? xm[((w * QUADS + quad) * 4 + lq) * 2 + 1] : 0.0f;
    const float ma = mh[quad], la = lh[quad];
    const float mm = fmaxf(ma, mb);
    const float wa = (la > 0.0f) ? exp2f(ma - mm) : 0.0f;
    const float wb2 = (lb > 0.0f) ? exp2f(mb - mm) : 0.0f;
    const float lt = la * wa + lb * wb2;
    const int hq = quad * 4 + lq;
    if (hq < p.gq) {
      float* orow = p.part_o + (prow + hq) * 128;
      float o[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        o[k] = wa != 0.0f ? wa * ov[quad][k] : 0.0f;
        if (G::HALVES == 2) o[k] += wb2 != 0.0f ? wb2 * src[k] : 0.0f;
      }
      if (BITS == 4) {
#pragma unroll
        for (int k = 0; k < 8; ++k) orow[16 * k + li] = o[k];
      } else {
#pragma unroll
        // (non-temporal: measured 0.3 µs faster per INT2 step; for INT4 the
        // same stores made the step 0.2 µs slower)
        for (int n = 0; n < 4; ++n) {
          __builtin_nontemporal_store(o[2 * n], orow + 32 * n + 2 * li);
          __builtin_nontemporal_store(o[2 * n + 1], orow + 32 * n + 2 * li + 1);
        }
      }
      if (li == 0) {
        if constexpr (BITS == 2) {
          __builtin_nontemporal_store(lt > 0.0f ? mm : -INFINITY, p.part_ml + 2 * (prow + hq));
          __builtin_nontemporal_store(lt, p.part_ml + 2 * (prow + hq) + 1);
        } else {
          p.part_ml[2 * (prow + hq)] = lt > 0.0f ? mm : -INFINITY;
          p.part_ml[2 * (prow + hq) + 1] = lt;
        }
      }
    }
  }
  KVSSD_STAMP(kStampStored);
}

template <int BITS, int QUADS, int QSPLIT, typename QT, int KG>
void launch_one(const StagedParams& prm, const SplitPlan& plan, int grid, hipStream_t s) {
  const uint32_t heads = pack_heads(prm.kv_heads, prm.gq, prm.table != nullptr);
  const DecodeTail rest{prm.valid,       prm.table,        prm.part_o,     prm.part_ml,
                        prm.query_heads, prm.num_blocks,   prm.scale_log2, plan.splits};
  const int split_arg = kInterleavedSplits<BITS> ? plan.splits : plan.blocks_per_split;
  hipLaunchKernelGGL((decode_staged_kernel<BITS, QUADS, QSPLIT, QT, KG>), dim3(grid), dim3(kThreads), 0, s, prm.query,
                     prm.pk, prm.pv, prm.sk, prm.sv, heads, prm.block_tokens, split_arg, prm.units, rest);
}

template <int BITS, int QUADS, int KG>
int launch_quads(const StagedParams& prm, const SplitPlan& plan, int grid, int dtype, hipStream_t s) {
  switch (dtype) {
    case KVSSD_DTYPE_F16:
      launch_one<BITS, QUADS, 1, _Float16, KG>(prm, plan, grid, s);
      break;
    case KVSSD_DTYPE_BF16:  // 8 significant bits: one fp16 part holds a normalised value exactly
      launch_one<BITS, QUADS, 1, uint16_t, KG>(prm, plan, grid, s);
      break;
    case KVSSD_DTYPE_F32:
    case KVSSD_DTYPE_F64:
      // (staged_wide never picks 8 kv heads for INT4 with two quads here)
      if constexpr (BITS == 4 && QUADS == 2 && KG == 8) return arg_error("no 8-kv-head form for this query");
      else if (dtype == KVSSD_DTYPE_F32) launch_one<BITS, QUADS, 2, float, KG>(prm, plan, grid, s);
      else launch_one<BITS, QUADS, 2, double, KG>(prm, plan, grid, s);
      break;
    default:
      return arg_error("unsupported query dtype");
  }
  return hip_status(hipGetLastError(), "decode_staged launch");
}

template <int KG>
int launch_kg(const StagedParams& prm, const SplitPlan& plan, int bits, int dtype, hipStream_t s) {
  const int grid = 8 * (prm.kv_heads / KG) * ((plan.splits + 7) / 8);
  const bool two = prm.gq > 4;
  if (bits == 4)
    return two ? launch_quads<4, 2, KG>(prm, plan, grid, dtype, s) : launch_quads<4, 1, KG>(prm, plan, grid, dtype, s);
  return two ? launch_quads<2, 2, KG>(prm, plan, grid, dtype, s) : launch_quads<2, 1, KG>(prm, plan, grid, dtype, s);
}

}  // namespace

bool staged_wide(const kvssd_decode_desc& d, int units) {
  // all 8 kv heads of a row per workgroup once the context gives every
  // workgroup at least one block: 2048 (kv head, split) work items, 256
  // workgroups.  Not for INT4 with two query quads and a two-part (fp32 /
  // fp64) query: that form needs more than 256 VGPRs with 8 kv heads (it
  // spilled), none with 4.
  const int gq = d.kv_heads > 0 ? d.query_heads / d.kv_heads : 0;
  const bool two_part = d.query_dtype == KVSSD_DTYPE_F32 || d.query_dtype == KVSSD_DTYPE_F64;
  if (d.bits == 4 && gq > 4 && two_part) return false;
  return d.head_dim == 128 && d.group_size == 32 && (d.bits == 2 || d.bits == 4) && d.kv_heads % 8 == 0 &&
         d.block_tokens % 128 == 0 && gq >= 1 && gq <= 8 && static_cast<long>(units) * d.kv_heads >= 2048;
}

bool staged_supported(const kvssd_decode_desc& d, std::string* why) {
  auto no = [&](const char* r) {
    if (why) *why = r;
    return false;
  };
  if (d.head_dim != 128) return no("head_dim must be 128");
  if (d.group_size != 32) return no("group_size must be 32");
  if (d.block_tokens % 128) return no("block_tokens must be a multiple of 128");
  if (d.kv_heads % 4) return no("kv_heads must be a multiple of 4");
  if (d.kv_heads > 0xFFFF) return no("kv_heads must be below 65536");
  const int units = d.num_selected > 0 ? d.num_selected : d.num_blocks;
  if (plan_splits(d, units).blocks_per_split > kMaxUnits) return no("too many blocks per split");
  const int gq = d.query_heads / d.kv_heads;
  if (gq < 1 || gq > 8) return no("at most 8 query heads per kv head");
  return true;
}

bool staged_aligned(const DecodeArgs& a) {
  auto ok = [&](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) % 16) == 0; };
  return ok(a.packed_k) && ok(a.packed_v) && ok(a.scales_k) && ok(a.scales_v);
}

int launch_staged(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts) {
  const kvssd_decode_desc& d = a.desc;
  StagedParams prm{};
  prm.query = a.query;
  prm.pk = a.packed_k;
  prm.pv = a.packed_v;
  prm.sk = reinterpret_cast<const uint8_t*>(a.scales_k);
  prm.sv = reinterpret_cast<const uint8_t*>(a.scales_v);
  prm.valid = a.valid;
  prm.table = a.table;
  prm.part_o = parts.o;
  prm.part_ml = parts.ml;
  prm.query_heads = d.query_heads;
  prm.kv_heads = d.kv_heads;
  prm.block_tokens = d.block_tokens;
  prm.num_blocks = d.num_blocks;
  prm.units = a.units;
  prm.gq = d.query_heads / d.kv_heads;
  prm.scale_log2 = static_cast<float>(d.sm_scale) * kLog2e;
  if (staged_wide(d, a.units)) return launch_kg<8>(prm, plan, d.bits, d.query_dtype, a.stream);
  return launch_kg<4>(prm, plan, d.bits, d.query_dtype, a.stream);
}

}  // namespace kvssd

#ifdef KVSSD_TIMELINE
// Instrumented build only (no declaration in include/kvssd_hip.h): copy the
// stamps out, or clear them before a run.
extern "C" __attribute__((visibility("default"))) int kvssd_hip_timeline_read(void* dst, size_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(dst, HIP_SYMBOL(kvssd_timeline_stamps), bytes, 0, hipMemcpyDeviceToHost));
}
extern "C" __attribute__((visibility("default"))) int kvssd_hip_timeline_clear(void) {
  void* ptr = nullptr;
  hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(kvssd_timeline_stamps));
  if (err == hipSuccess) err = hipMemset(ptr, 0, sizeof(kvssd_timeline_stamps));
  return static_cast<int>(err);
}
#endif
