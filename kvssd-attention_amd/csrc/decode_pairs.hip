// Pair-owned LDS-staged matrix-core decode kernel for gfx950: INT4 codes,
// head_dim 128, group_size 32, at most 4 query heads per kv head,
// kv_heads % 4 == 0, block_tokens % (stage tokens) == 0.
//
// Same semantics as the general kernel (ReferenceAttentionBackend.run,
// src/kvssd/backends/reference.py:22-50; element addressing of
// csrc/fused_decode.cu:50-56).
//
// Work split.  A workgroup of 8 waves owns 2P consecutive kv heads (P kv-head
// pairs, P = 2 or 4) and one split (a range of attended blocks).  It walks
// the split in stages of 32 * (8 / P) tokens; wave (pair, slice) computes both
// kv heads of its pair over tokens 32 slice .. 32 slice + 31 of every stage,
// and the slices meet in LDS at the end, so each workgroup writes one partial
// per query head of its kv heads.
//
// Ownership.  The packed K (or V) rows of a kv-head pair and one token are
// 128 contiguous bytes, one whole cache line, so every wave copies exactly
// the lines it reads: its own K, V and scale rows, HBM -> LDS with
// global_load_lds (16 bytes per lane for codes, 4 for scales), into two
// buffers of its own.  No wave waits for another inside the loop: the only
// synchronisation is the wave's own vmcnt, which leaves the next stage's
// copies in flight while the current stage is computed.
//
// LDS per wave and stage (9 KB): K rows [32 tokens][8 chunks of 16 B] at 0,
// V rows at 4096, K scales [32 tokens][2 heads x 4 fp16] at 8192, V scales at
// 8704.  Chunk c of a token holds kv head c >> 2, dims 32(c & 3) .. +31; it
// sits in slot c ^ f(t) of token t's 128 bytes, f(t) = (t & 3) |
// (((t >> 2) ^ (t >> 4)) & 1) << 2, so that the K operand reads (8 lanes =
// 8 consecutive tokens) and the V transpose reads (16 lanes = 8 tokens x 2
// halves, see below) hit distinct banks.
//
// Math per wave and stage (one kv head hh of the pair at a time, both
// interleaved): as decode_staged.hip (shared code in staged_ops.hpp) -- QK
// with the query operand of head hh
// against K tiles of 16 tokens, fp16-operand scores against the K scales,
// per-stage running softmax in log2 units, W = p * scale_v in fp16 through
// LDS, PV with the transposed V codes from ds_read_b64_tr_b4.
// Token <-> MFMA K slot (PV, shared by A and B): lane group q, slot s ->
// token T(q, s) = 4q + (s >> 1) + 16(s & 1).  A transpose read of lane group
// q addresses, in row r = li & 7, token 4q + (r & 3) + 16(r >> 2), half
// li >> 3 of the chunk (dims +0 / +16): its dword 0 is the A operand of one
// 16-dim tile, dword 1 that of the next.  W of head hh lives in the wave's
// consumed K rows at 1024 hh, [row q][column c][8 slots] with the 16-byte
// column slot c ^ q.
#include "staged_ops.hpp"

namespace kvssd {
namespace {

constexpr int kPWaves = 8;
constexpr int kPThreads = 64 * kPWaves;
constexpr int kSliceTok = 32;  // tokens per wave and stage
constexpr int kRowBytes = 128; // packed K (or V) bytes of a kv-head pair and token
constexpr int kBufK = 0;
constexpr int kBufV = 4096;
constexpr int kBufSK = 8192;
constexpr int kBufSV = 8704;
constexpr int kBufBytes = 9216;              // one stage of one wave
constexpr int kWaveBytes = 2 * kBufBytes;    // double buffer
constexpr int kPMaxUnits = 2048;             // attended blocks per split (block list kept in LDS)
constexpr int kPCopies = 12;                 // copy instructions per wave and stage
constexpr int kPLds = kPWaves * kWaveBytes + kPMaxUnits * 8;
static_assert(kPLds <= 160 * 1024, "LDS budget");

struct PairParams {
  const void* query;
  const uint8_t* pk;
  const uint8_t* pv;
  const uint8_t* sk;  // fp16 scales as bytes
  const uint8_t* sv;
  const int32_t* valid;
  const int32_t* table;
  float* part_o;
  float* part_ml;
  int query_heads, kv_heads, block_tokens, num_blocks, units, splits, blocks_per_split, gq;
  float scale_log2;  // sm_scale * log2(e)
};

__device__ __forceinline__ int pair_swz(int t) { return (t & 3) | ((((t >> 2) ^ (t >> 4)) & 1) << 2); }

// byte of chunk c of slice token t inside a K or V region
__device__ __forceinline__ int row_byte(int t, int c) { return kRowBytes * t + 16 * (c ^ pair_swz(t)); }


// Per-lane byte offsets, relative to the stage's first row of the pair, of the
// wave's copies: code instruction j covers tokens 8j .. 8j+7 (LDS slot
// lane & 7 of token 8j + lane/8 receives chunk slot ^ f(t)), scale instruction
// j covers tokens 16j .. 16j+15 (dword lane & 3 of token 16j + lane/4).
struct PairCopies {
  uint32_t kv[4];
  uint32_t sc[2];
};

__device__ __forceinline__ PairCopies make_pair_copies(int lane, int kv_heads) {
  PairCopies cm;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ pair_swz(t);
    cm.kv[j] = static_cast<uint32_t>(t * kv_heads * 64 + 16 * c);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = 16 * j + (lane >> 2);
    cm.sc[j] = static_cast<uint32_t>(t * kv_heads * 8 + 4 * (lane & 3));
  }
  return cm;
}

// row0 = (block * block_tokens + first token) * kv_heads + first kv head of the pair
__device__ __forceinline__ void issue_pair_stage(const PairParams& p, uint32_t buf, long row0, const PairCopies& cm) {
  const uint8_t* kb = p.pk + row0 * 64;
  const uint8_t* vb = p.pv + row0 * 64;
  const uint8_t* skb = p.sk + row0 * 8;
  const uint8_t* svb = p.sv + row0 * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) dma16<true>(kb, cm.kv[j], buf + kBufK + 1024u * j);
#pragma unroll
  for (int j = 0; j < 2; ++j) dma4(skb, cm.sc[j], buf + kBufSK + 256u * j);
#pragma unroll
  for (int j = 0; j < 4; ++j) dma16<true>(vb, cm.kv[j], buf + kBufV + 1024u * j);
#pragma unroll
  for (int j = 0; j < 2; ++j) dma4(svb, cm.sc[j], buf + kBufSV + 256u * j);
}

// vmcnt waits with a compiler memory barrier: no LDS access moves across them
__device__ __forceinline__ void wait_all_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_all_but_one_stage() {
  static_assert(kPCopies == 12, "vmcnt immediate below");
  asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
}

struct PairState {
  float m_run[2], l_run[2];  // per kv head of the pair, of query head lq
  f32x4 acc[2][8];
  f32x4 corr[2];
};

// One stage of one wave: tokens 0 .. hv-1 of its 32-token slice are valid
// (hv may be <= 0 or > 32).
template <int QSPLIT>
__device__ __forceinline__ void pair_stage(uint8_t* buf, int hv, int li, int lq, const Masks& mk, float wf,
                                           const QueryOps<1, QSPLIT> (&qo)[2], const u32x4& offa, PairState& st) {
  // ------------------------------------------------------------ LDS reads
  uint32_t kraw[2][2][4];  // [head][tile][word]
  u32x4 skw[2], svw[2];    // [tile]: words 0-1 head 0, 2-3 head 1
#pragma unroll
  for (int tau = 0; tau < 2; ++tau) {
    const int t = 16 * tau + li;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(buf + kBufK + row_byte(t, 4 * hh + lq));
#pragma unroll
      for (int i = 0; i < 4; ++i) kraw[hh][tau][i] = r[i];
    }
    skw[tau] = *reinterpret_cast<const u32x4*>(buf + kBufSK + 16 * t);
    svw[tau] = *reinterpret_cast<const u32x4*>(buf + kBufSV + 16 * t);
  }
  const int rr = li & 7;
  const int t_tr = 4 * lq + (rr & 3) + 16 * (rr >> 2);
  i32x2 tr[2][4];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int np = 0; np < 4; ++np) tr[hh][np] = lds_read_tr4(buf, kBufV + row_byte(t_tr, 4 * hh + np) + 8 * (li >> 3));
  // ---------------------------------------------------------------- QK
  f32x4 cc[2][2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) cc[hh][tau] = qo[hh].qcorr[0];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    u32x4 b[2][2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int tau = 0; tau < 2; ++tau) b[hh][tau] = unpack4(kraw[hh][tau][m], mk);
#pragma unroll
    for (int sp = 0; sp < QSPLIT; ++sp)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int tau = 0; tau < 2; ++tau) cc[hh][tau] = mfma16(qo[hh].qa[0][sp][m], b[hh][tau], cc[hh][tau]);
  }
  bool ok[2];
  float score[2][2];
#pragma unroll
  for (int tau = 0; tau < 2; ++tau) {
    ok[tau] = 16 * tau + li < hv;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const f32x4 c = cc[hh][tau];
      const uint32_t w0 = skw[tau][2 * hh], w1 = skw[tau][2 * hh + 1];
      float raw = __builtin_fmaf(half_lo(w0), c[0], 0.0f);
      raw = __builtin_fmaf(half_hi(w0), c[1], raw);
      raw = __builtin_fmaf(half_lo(w1), c[2], raw);
      raw = __builtin_fmaf(half_hi(w1), c[3], raw);
      score[hh][tau] = ok[tau] ? raw * qo[hh].kscale[0] : -INFINITY;
    }
  }
  // --------------------------------------------- V operands (no softmax dep)
  u32x4 va[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int np = 0; np < 4; ++np)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) va[hh][2 * np + hf] = unpack4(static_cast<uint32_t>(tr[hh][np][hf]), mk);
  // --------------------------------------------------------------- softmax
  uint8_t* wreg = buf + kBufK;  // W of head hh at 1024 hh (K rows already read)
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const float mx = row_max16_of(score[hh][0], score[hh][1], score[hh][1], score[hh][1]);
    const float m_new = fmaxf(st.m_run[hh], mx);
    const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(st.m_run[hh] - m_new);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    st.m_run[hh] = m_new;
    const float p0 = __builtin_amdgcn_exp2f(score[hh][0] - m_use);
    const float p1 = __builtin_amdgcn_exp2f(score[hh][1] - m_use);
    st.l_run[hh] = st.l_run[hh] * alpha + (p0 + p1);
    // W[t, (lq, g)] = p * scale_v[t, hh, g] * F(slot)/64; masked tokens carry
    // scale 0.  Token li -> (row li >> 2, slot 2 (li & 3)), token 16 + li ->
    // the next slot; both slots have F = 1024 iff li is even (wf = 16).
    const float w0 = p0 * wf, w1 = p1 * wf;
    const uint32_t a01 = ok[0] ? svw[0][2 * hh] : 0u, a23 = ok[0] ? svw[0][2 * hh + 1] : 0u;
    const uint32_t b01 = ok[1] ? svw[1][2 * hh] : 0u, b23 = ok[1] ? svw[1][2 * hh + 1] : 0u;
    uint32_t wv[4];
    wv[0] = pack_half2(static_cast<_Float16>(w0 * half_lo(a01)), static_cast<_Float16>(w1 * half_lo(b01)));
    wv[1] = pack_half2(static_cast<_Float16>(w0 * half_hi(a01)), static_cast<_Float16>(w1 * half_hi(b01)));
    wv[2] = pack_half2(static_cast<_Float16>(w0 * half_lo(a23)), static_cast<_Float16>(w1 * half_lo(b23)));
    wv[3] = pack_half2(static_cast<_Float16>(w0 * half_hi(a23)), static_cast<_Float16>(w1 * half_hi(b23)));
    const int q = li >> 2;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<uint32_t*>(wreg + 1024 * hh + 256 * q + 16 * ((4 * lq + g) ^ q) + 4 * (li & 3)) = wv[g];
    // rescale the PV state of column head li/4 by that head's alpha (alpha
    // is uniform over each row: head h in lanes 16h .. 16h+15)
    const RowValue a_pv = row_value(alpha, li >> 2);
    if (a_pv.any_not_one) {
#pragma unroll
      for (int n = 0; n < 8; ++n) st.acc[hh][n] *= a_pv.v;
      st.corr[hh] *= a_pv.v;
    }
  }
  // -------------------------------------------------------------------- PV
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const u32x4 wb = *reinterpret_cast<const u32x4*>(wreg + 1024 * hh + 256 * lq + 16 * (li ^ lq));
#pragma unroll
    for (int n = 0; n < 8; ++n) st.acc[hh][n] = mfma16(va[hh][n], wb, st.acc[hh][n]);
    // sum over tokens of W * OFF per column, through the matrix core
    st.corr[hh] = mfma16(offa, wb, st.corr[hh]);
  }
}

template <int P, int QSPLIT, typename QT>
__global__ __launch_bounds__(kPThreads) void decode_pairs_kernel(PairParams p) {
  constexpr int S = kPWaves / P;             // token slices per stage
  constexpr int kStageTok = kSliceTok * S;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kPLds];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int pr = wave % P;
  const int slice = wave / P;
  const int li = lane & 15;
  const int lq = lane >> 4;

  // workgroup -> (split, group of 2P kv heads).  Consecutive workgroup ids go
  // to different XCDs (round robin over 8); every group of split s gets an id
  // with id % 8 == s % 8, so they share one XCD and its L2: they read
  // complementary parts of the same 128-byte lines of the scale rows.
  const int groups = p.kv_heads / (2 * P);
  const int xcd = blockIdx.x & 7;
  const int rest = blockIdx.x >> 3;
  const int grp = rest % groups;
  const int split = (rest / groups) * 8 + xcd;
  if (split >= p.splits) return;  // padding ids of the last round
  const int u_begin = split * p.blocks_per_split;
  const int u_end = min(p.units, u_begin + p.blocks_per_split);
  const int kvh = grp * 2 * P + 2 * pr;  // first kv head of the wave's pair

  uint8_t* wlds = lds + wave * kWaveBytes;
  const uint32_t wlds_a = lds_addr(wlds);
  const PairCopies cm = make_pair_copies(lane, p.kv_heads);
  auto row0 = [&](const Cursor& c) {
    return (static_cast<long>(c.blk) * p.block_tokens + c.sb0 + kSliceTok * slice) * p.kv_heads + kvh;
  };

  // The first stage's copies go out before anything else: the split's first
  // attended block, tokens 0 .. kStageTok-1 (one scalar read with a block
  // table).  If that block holds no valid token they are simply not used.
  bool spec = false;
  if (u_begin < u_end) {
    const Cursor c0{0, __builtin_amdgcn_readfirstlane(p.table ? p.table[u_begin] : u_begin), 0, 0};
    if (c0.blk >= 0 && c0.blk < p.num_blocks) {
      issue_pair_stage(p, wlds_a, row0(c0), cm);
      spec = true;
    }
  }

  // the query loads go out next: they complete in issue order, right after
  // the first stage's copies, instead of a round trip after them
  const QueryRaw<1> qraw0 = coop_query_load<4, 1, QT>(p.query, p.gq, kvh * p.gq, lane);
  const QueryRaw<1> qraw1 = coop_query_load<4, 1, QT>(p.query, p.gq, (kvh + 1) * p.gq, lane);

  // the split's (block id, clamped valid count) list, read once into LDS
  int* units = reinterpret_cast<int*>(lds + kPWaves * kWaveBytes);
  const int n_units = max(0, u_end - u_begin);  // <= kPMaxUnits, checked on the host
  for (int i = threadIdx.x; i < n_units; i += kPThreads) {
    const int blk = p.table ? p.table[u_begin + i] : u_begin + i;
    units[2 * i] = blk;
    units[2 * i + 1] = (blk < 0 || blk >= p.num_blocks) ? 0 : clamp_valid(p.valid[blk], p.block_tokens);
  }
  __syncthreads();

  Cursor cur{-1, 0, 0, -kStageTok};
  bool have = next_stage<kStageTok>(cur, units, n_units);
  if (have && !(spec && cur.u == 0 && cur.sb0 == 0)) {
    // the first valid stage is elsewhere: let the early copies land (they
    // target the same LDS bytes), then load the right ones
    wait_all_copies();
    issue_pair_stage(p, wlds_a, row0(cur), cm);
  }

  // query operands, through the wave's second buffer (its first copies go
  // out in the loop, after these LDS accesses are done)
  QueryOps<1, QSPLIT> qo[2];
  static_assert(2 * coop_scratch_bytes<1> <= kBufBytes, "query scratch fits a buffer");
  coop_query_build<4, 1, QSPLIT>(qo[0], qraw0, p.scale_log2, lane, wlds + kBufBytes);
  coop_query_build<4, 1, QSPLIT>(qo[1], qraw1, p.scale_log2, lane, wlds + kBufBytes + coop_scratch_bytes<1>);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // masks in VGPRs: p.units >= 1, so (lane & (p.units >> 30)) is 0 but opaque
  const Masks mk = make_masks(static_cast<uint32_t>(lane) & static_cast<uint32_t>(p.units >> 30));
  const u32x4 offa = off_operand4();
  const float wf = (li & 1) == 0 ? 16.0f : 1.0f;  // F/64 of this lane's W slots

  PairState st;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    st.m_run[hh] = -INFINITY;
    st.l_run[hh] = 0.0f;
#pragma unroll
    for (int n = 0; n < 8; ++n) st.acc[hh][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    st.corr[hh] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // --------------------------------------- double-buffered, per-wave stages
  // The stage after the current one is looked up a step ahead; its copies go
  // out before the current stage is computed, and the wait leaves exactly
  // them in flight (copies complete in issue order).
  Cursor nxt = cur;
  bool have_n = have && next_stage<kStageTok>(nxt, units, n_units);
  int buf = 0;
  while (have) {
    if (have_n) {
      issue_pair_stage(p, wlds_a + static_cast<uint32_t>((buf ^ 1) * kBufBytes), row0(nxt), cm);
      wait_all_but_one_stage();
    } else {
      wait_all_copies();
    }
    // (a slice past the block's valid tokens computes too: every token is
    // masked, so p = 0, alpha = 1 and the state is unchanged; a branch here
    // costs a copy of every accumulator per stage)
    const int hv = cur.vb - cur.sb0 - kSliceTok * slice;
    pair_stage<QSPLIT>(wlds + buf * kBufBytes, hv, li, lq, mk, wf, qo, offa, st);
    cur = nxt;
    have = have_n;
    if (have) have_n = next_stage<kStageTok>(nxt, units, n_units);
    buf ^= 1;
  }

  // -------------------------------------------------------------- epilogue
  // out = 64 (C - corr) per column; lane (li, lq): column (head li/4, group
  // li%4), rows = dims 16n + 4lq + i of tiles n = 2g, 2g+1.
  float ov[2][8], mh[2], lh[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int g = li & 3;
    const float cr = st.corr[hh][0];
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
      if (gg == g) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ov[hh][i] = 64.0f * (st.acc[hh][2 * gg][i] - cr);
          ov[hh][4 + i] = 64.0f * (st.acc[hh][2 * gg + 1][i] - cr);
        }
      }
    }
    // (m, l) of head li/4 (the QK layout keeps head lq in lanes 16lq..16lq+15)
    const float l_tot = row_sum16(st.l_run[hh]);
    mh[hh] = __shfl(st.m_run[hh], (li >> 2) << 4, kWave);
    lh[hh] = __shfl(l_tot, (li >> 2) << 4, kWave);
  }
  // slices 1..S-1 hand (o, m, l) to slice 0 through LDS
  float* xo = reinterpret_cast<float*>(lds);           // [slice-1][pair][hh][lane][8]
  float* xm = xo + (S - 1) * P * 2 * 64 * 8;           // [slice-1][pair][hh][lane][2]
  wait_all_copies();  // no copy of this wave is still writing LDS
  __syncthreads();    // every wave is done with its stage buffers
  if (slice > 0) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int slot = (((slice - 1) * P + pr) * 2 + hh) * 64 + lane;
#pragma unroll
      for (int i = 0; i < 8; ++i) xo[slot * 8 + i] = ov[hh][i];
      xm[slot * 2] = mh[hh];
      xm[slot * 2 + 1] = lh[hh];
    }
  }
  __syncthreads();
  if (slice > 0) return;
  const long prow = static_cast<long>(split) * p.query_heads;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    float mm = lh[hh] > 0.0f ? mh[hh] : -INFINITY;
#pragma unroll
    for (int s = 1; s < S; ++s) {
      const int slot = (((s - 1) * P + pr) * 2 + hh) * 64 + lane;
      if (xm[slot * 2 + 1] > 0.0f) mm = fmaxf(mm, xm[slot * 2]);
    }
    const float w0 = lh[hh] > 0.0f ? exp2f(mh[hh] - mm) : 0.0f;
    float lt = lh[hh] * w0;
    f32x4 o0, o1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o0[i] = w0 != 0.0f ? w0 * ov[hh][i] : 0.0f;
      o1[i] = w0 != 0.0f ? w0 * ov[hh][4 + i] : 0.0f;
    }
#pragma unroll
    for (int s = 1; s < S; ++s) {
      const int slot = (((s - 1) * P + pr) * 2 + hh) * 64 + lane;
      const float ls = xm[slot * 2 + 1];
      const float ws = ls > 0.0f ? exp2f(xm[slot * 2] - mm) : 0.0f;
      lt += ls * ws;
      if (ws != 0.0f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o0[i] += ws * xo[slot * 8 + i];
          o1[i] += ws * xo[slot * 8 + 4 + i];
        }
      }
    }
    const int hcol = li >> 2;
    if (hcol < p.gq) {
      const long row = prow + (kvh + hh) * p.gq + hcol;
      float* orow = p.part_o + row * 128;
      const int g = li & 3;
      *reinterpret_cast<f32x4*>(orow + 32 * g + 4 * lq) = o0;
      *reinterpret_cast<f32x4*>(orow + 32 * g + 16 + 4 * lq) = o1;
      if (lq == 0 && g == 0) {
        p.part_ml[2 * row] = lt > 0.0f ? mm : -INFINITY;
        p.part_ml[2 * row + 1] = lt;
      }
    }
  }
}

template <int P, int QSPLIT, typename QT>
void launch_pairs_one(const PairParams& prm, int grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_pairs_kernel<P, QSPLIT, QT>), dim3(grid), dim3(kPThreads), 0, s, prm);
}

template <int P>
int launch_pairs_p(const PairParams& prm, int grid, int dtype, hipStream_t s) {
  switch (dtype) {
    case KVSSD_DTYPE_F16:
      launch_pairs_one<P, 1, _Float16>(prm, grid, s);
      break;
    case KVSSD_DTYPE_BF16:
      launch_pairs_one<P, 2, uint16_t>(prm, grid, s);
      break;
    case KVSSD_DTYPE_F32:
      launch_pairs_one<P, 2, float>(prm, grid, s);
      break;
    case KVSSD_DTYPE_F64:
      launch_pairs_one<P, 2, double>(prm, grid, s);
      break;
    default:
      return arg_error("unsupported query dtype");
  }
  return hip_status(hipGetLastError(), "decode_pairs launch");
}

// kv-head pairs per workgroup for a shape
int pairs_per_group(const kvssd_decode_desc&) { return 2; }

}  // namespace

bool pairs_supported(const kvssd_decode_desc& d, std::string* why) {
  auto no = [&](const char* r) {
    if (why) *why = r;
    return false;
  };
  if (d.bits != 4) return no("bits must be 4");
  if (d.head_dim != 128) return no("head_dim must be 128");
  if (d.group_size != 32) return no("group_size must be 32");
  if (d.kv_heads % 4) return no("kv_heads must be a multiple of 4");
  const int stage_tok = kSliceTok * (kPWaves / pairs_per_group(d));
  if (d.block_tokens % stage_tok) return no("block_tokens must be a multiple of the stage");
  const int units = d.num_selected > 0 ? d.num_selected : d.num_blocks;
  if (plan_splits(d, units).blocks_per_split > kPMaxUnits) return no("too many blocks per split");
  const int gq = d.query_heads / d.kv_heads;
  if (gq < 1 || gq > 4) return no("at most 4 query heads per kv head");
  return true;
}

int launch_pairs(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts) {
  const kvssd_decode_desc& d = a.desc;
  PairParams prm{};
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
  prm.splits = plan.splits;
  prm.blocks_per_split = plan.blocks_per_split;
  prm.gq = d.query_heads / d.kv_heads;
  prm.scale_log2 = static_cast<float>(d.sm_scale) * kLog2e;
  const int P = pairs_per_group(d);
  const int grid = 8 * (d.kv_heads / (2 * P)) * ((plan.splits + 7) / 8);
  return P == 4 ? launch_pairs_p<4>(prm, grid, d.query_dtype, a.stream)
                : launch_pairs_p<2>(prm, grid, d.query_dtype, a.stream);
}

}  // namespace kvssd
