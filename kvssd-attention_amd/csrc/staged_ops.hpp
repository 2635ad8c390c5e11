// Device helpers of the LDS-staged matrix-core decode kernel
// (decode_staged.hip): operand types, the global -> LDS
// copies, the in-register code -> fp16 unpack, the QK query operands and the
// stage cursor.
#pragma once

#include "decode.hpp"

namespace kvssd {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------ small helpers

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c, 0,
                                                0, 0);
}

__device__ __forceinline__ uint32_t pack_half2(_Float16 lo, _Float16 hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

// (fp16(a0 * b0), fp16(a1 * b1)) as one fp16 pair: written as fused
// multiply-adds of +0 into a two-element vector, the compiler forms each half
// with one v_fma_mix{lo,hi}_f16 (products of an fp32 and an fp16 value).
__device__ __forceinline__ uint32_t wpair(float a0, float b0, float a1, float b1) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const half2_t v = {static_cast<_Float16>(__builtin_fmaf(a0, b0, 0.0f)),
                     static_cast<_Float16>(__builtin_fmaf(a1, b1, 0.0f))};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float half_lo(uint32_t x) { return half_bits_to_float(static_cast<uint16_t>(x & 0xFFFFu)); }
__device__ __forceinline__ float half_hi(uint32_t x) { return half_bits_to_float(static_cast<uint16_t>(x >> 16)); }

// LDS byte address of a pointer into a __shared__ array
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t*)p));
}

// ds_read_b64_tr_b4: within each group of 16 lanes, lane j receives nibble j of
// the 8 bytes every lane of the group addressed, lane r's nibble landing in
// bits 4r..4r+3 (a 16x16 nibble transpose).
__device__ __forceinline__ i32x2 lds_read_tr4(const uint8_t* lds, int offset) {
  typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
  return __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2*)(lds + offset));
}

// One global -> LDS copy instruction: lane i's 16 bytes from sbase + voff land
// at LDS byte lds_dst + 16 i.  Issued from asm so that the compiler does not
// treat it as a pending write to every LDS location: in its intrinsic form the
// compiler waits for all outstanding copies (i.e. the next stage's prefetch)
// before any LDS read it cannot tell apart from them.  The copies' completion
// is awaited explicitly (vmcnt) before a stage is read.
// M0 is a reserved register the compiler does not track through asm clobbers;
// the kernels using these copies have no other M0 user (no compiler-issued
// LDS copies, dynamic register indexing or messages), so the asm owns it.
// NT: non-temporal hint, for the code arrays, read once per decode (streaming
// reads measured ~8% faster with it).  Scale rows keep the default policy:
// with 4 kv heads per workgroup the split's other workgroup reads the rest of
// each 128-byte scale line from the same L2, and with 8 the hint on the scale
// copies measured slower as well (+0.7 us on a 128K-token INT4 decode).
template <bool NT>
__device__ __forceinline__ void dma16(const uint8_t* sbase, uint32_t voff, uint32_t lds_dst) {
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase),
                 "s"(lds_dst)
                 : "memory");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_dst)
                 : "memory");
}

// As dma16 with 4 bytes per lane: lane i's dword lands at LDS byte lds_dst + 4 i.
__device__ __forceinline__ void dma4(const uint8_t* sbase, uint32_t voff, uint32_t lds_dst) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_dst)
               : "memory");
}

// ---------------------------------------------------------- code -> fp16 ---
//
// A code c placed at bit b (b + width <= 10) of an fp16 whose exponent field
// is that of 1.0 reads as v = 1 + c/F with F = 2^(10 - b), and
// (c - mid) = F (v - OFF), OFF = 1 + mid/F.  Codes stay in the normal range
// (codes left in place as fp16 subnormals would save shifts, but the matrix
// core does not multiply subnormal operands exactly against operands of wide
// exponent range).  One shift per distinct distance plus one AND-OR per fp16
// pair; the masks live in VGPRs (a three-operand VALU op may read only one
// scalar).  The factor F(s) of each MFMA K slot is exact (a power of two) and
// is carried by the other operand: by the query in QK, by W in PV.
struct Masks {
  uint32_t m03;  // bits 0-3 of both halves (INT4, F = 1024)
  uint32_t m47;  // bits 4-7 (INT4, F = 64)
  uint32_t m45;  // bits 4-5 (INT2, F = 64)
  uint32_t m67;  // bits 6-7 (INT2, F = 16)
  uint32_t m89;  // bits 8-9 (INT2, F = 4)
};

__device__ __forceinline__ Masks make_masks(uint32_t opaque_zero) {
  return Masks{0x000F000Fu | opaque_zero, 0x00F000F0u | opaque_zero, 0x00300030u | opaque_zero,
               0x00C000C0u | opaque_zero, 0x03000300u | opaque_zero};
}

// (x & m) | 1.0-pairs as one v_bitop3_b32 (truth table 0xEA = (a & b) | c): a
// compiler builtin, so the hazard recognizer sees it like any VALU op.
__device__ __forceinline__ uint32_t ao(uint32_t x, uint32_t m) { return __builtin_amdgcn_bitop3_b32(x, m, kF16One2, 0xEA); }

// INT4 word x (nibbles n0..n7, n_i at bits 4i): fp16 slots s0..s7 hold
// n0, n4, n1, n5, n2, n6, n3, n7 (slot s <-> nibble (s>>1) + 4(s&1)) with one
// shift: n0, n4, n2, n6 stay at bits 0-3 of their half (F = 1024), n1, n5,
// n3, n7 at bits 4-7 (F = 64), i.e. F(s) = 1024 for s in {0, 1, 4, 5}.  The
// same routine serves K rows (nibble = dim) and transpose-read V words
// (nibble = token row).
__device__ __forceinline__ u32x4 unpack4(uint32_t x, const Masks& k) {
  const uint32_t y = x >> 8;
  return u32x4{ao(x, k.m03), ao(x, k.m47), ao(y, k.m03), ao(y, k.m47)};
}

// INT4 slot s holds its code at F = 1024 (else F = 64)
constexpr bool fine_slot4(int s) { return ((s >> 1) & 1) == 0; }

// INT2 K word x (codes c0..c15, c_j at bits 2j): register i of MFMA step
// parity o (0 or 1) holds the pair (c_j, c_{j+8}), j = int2_code(o, i), in
// its two halves (slot s = 2i + hi holds c_{j + 8 hi}).  Every code lands at
// bits 4-5 (F = 64), 6-7 (F = 16) or 8-9 (F = 4) of its half: c2..c4 are
// there already, c5..c7 after x >> 6, c0 and c1 after x << 6 -- two shifts
// per word.  The offset term the accumulator carries grows with F, and its
// fp32 rounding with it; a score sums 128 dims only, so F = 64 costs nothing
// measurable (c0 and c1 left at F = 1024 and 256 would save one more shift).
__host__ __device__ constexpr int int2_code(int o, int i) { return (2 + 4 * o + i) & 7; }
// c_j sits at bit 4 + 2 ((j + 1) mod 3) of its half
__host__ __device__ constexpr float int2_f(int j) { return static_cast<float>(64 >> (2 * ((j + 1) % 3))); }

__device__ __forceinline__ u32x4 unpack2(uint32_t x, int o, const Masks& k) {
  const uint32_t r = x >> 6;
  if (o == 0) return u32x4{ao(x, k.m45), ao(x, k.m67), ao(x, k.m89), ao(r, k.m45)};
  const uint32_t l = x << 6;
  return u32x4{ao(r, k.m67), ao(r, k.m89), ao(l, k.m67), ao(l, k.m89)};
}

// INT2 transpose-read word x (nibble rho = codes of dims 2j, 2j+1 of token
// row rho; slot s <-> row (s>>1) + 4(s&1)): parity 0 takes the even-dim code
// (bits 4rho..4rho+1) to bits 8-9 (F = 4), parity 1 the odd one to bits 6-7
// (F = 16); the shifts (8, 4, -4, -8) serve both.  (Parity 0 at bits 4-5
// would need one shift fewer per word, but at F = 64 the offset the
// accumulator carries over a split's tokens grows 16-fold, and with it the
// fp32 rounding: measured 4x the output error on outlier-heavy values.)
__device__ __forceinline__ u32x4 unpack2_tr(uint32_t x, int parity, const Masks& k) {
  if (parity == 0) return u32x4{ao(x << 8, k.m89), ao(x << 4, k.m89), ao(x, k.m89), ao(x >> 4, k.m89)};
  return u32x4{ao(x << 4, k.m67), ao(x, k.m67), ao(x >> 4, k.m67), ao(x >> 8, k.m67)};
}

// QK: the query operand of MFMA step m's K slot s carries F / G, so every
// product is q * v * F / G, and the accumulator starts at -sum q' OFF;
// then C = sum q (c - mid) / G (mid = 8 for INT4, 2 for INT2: OFF = 1 + mid/F).
template <int BITS>
constexpr float kQkG = BITS == 4 ? 64.0f : 4.0f;
template <int BITS>
__device__ __forceinline__ float slot_f(int m, int s) {
  if (BITS == 4) return fine_slot4(s) ? 1024.0f : 64.0f;
  return int2_f(int2_code(m & 1, s >> 1));
}
template <int BITS>
__device__ __forceinline__ float qk_factor(int m, int s) {
  return slot_f<BITS>(m, s) / kQkG<BITS>;
}
template <int BITS>
__device__ __forceinline__ float qk_off(int m, int s) {
  return 1.0f + (BITS == 4 ? 8.0f : 2.0f) / slot_f<BITS>(m, s);
}

// dim of QK MFMA m's slot s for lane group q
template <int BITS>
__device__ __forceinline__ int qk_dim(int m, int q, int s) {
  if (BITS == 4) return 32 * q + 8 * m + (s >> 1) + 4 * (s & 1);
  return 32 * q + 16 * (m >> 1) + int2_code(m & 1, s >> 1) + 8 * (s & 1);
}

// PV: INT2 V codes sit at one position per output tile (parity 0: F = 4,
// parity 1: F = 16), so out = F (C - sum_t W OFF); the correction operand
// holds one OFF per column (its slots alike), parity 0's in columns 0-7 and
// parity 1's in 8-15, so one MFMA per K step yields both sums.  INT4 V codes sit at F(s) per K
// slot; W of slot s carries F(s)/64, the correction operand OFF(s), and
// out = 64 (C - sum_t W' OFF).
__device__ __forceinline__ u32x4 off_operand(float off) {
  const _Float16 h = static_cast<_Float16>(off);
  const uint32_t w = pack_half2(h, h);
  return u32x4{w, w, w, w};
}
__device__ __forceinline__ u32x4 off_operand4() {
  const _Float16 f = static_cast<_Float16>(qk_off<4>(0, 0)), c = static_cast<_Float16>(qk_off<4>(0, 2));
  const uint32_t wf = pack_half2(f, f), wc = pack_half2(c, c);
  return u32x4{wf, wc, wf, wc};
}

// ---------------------------------------------------------- row reductions
// max over the 16 lanes of each row of max(a, b, c, d) (pass b = c = d = a
// for fewer inputs), in every lane: v_max_f32 with DPP row rotations.  (The
// compiler's form of a DPP reduction moves the operand through a separate DPP
// mov and canonicalises it: four instructions a step.)  s_nop 1 before each
// DPP read covers the VALU-write -> DPP-read hazard (two wait states);
// nothing in the sequence involves the matrix core.
__device__ __forceinline__ float row_max16_of(float a, float b, float c, float d) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3\n\t"
      "v_max_f32 %0, %0, %4\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:2 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:1 row_mask:0xf bank_mask:0xf"
      : "=&v"(r)
      : "v"(a), "v"(b), "v"(c), "v"(d));
  return r;
}

// A value uniform over each 16-lane row (row h = lanes 16h .. 16h+15), read
// by every lane for row hsel, and whether any row differs from 1.0 (scalar):
// the four row values go through SGPRs instead of an LDS permute.
struct RowValue {
  float v;
  bool any_not_one;
};
__device__ __forceinline__ RowValue row_value(float x, int hsel) {
  constexpr int kOne = 0x3F800000;
  const int a0 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 0);
  const int a1 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 16);
  const int a2 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 32);
  const int a3 = __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 48);
  const bool any = ((a0 ^ kOne) | (a1 ^ kOne) | (a2 ^ kOne) | (a3 ^ kOne)) != 0;
  const int v = hsel == 0 ? a0 : hsel == 1 ? a1 : hsel == 2 ? a2 : a3;
  return RowValue{__builtin_bit_cast(float, v), any};
}

// ---------------------------------------------------------------- cursor ---
struct Cursor {
  int u, blk, vb, sb0;
};

// Advance to the next stage (STAGE_TOK tokens) holding at least one valid token; false at the
// end of the split.  units[2i] / units[2i+1] = block id / clamped valid count
// of the split's i-th attended block (LDS).  Wave-uniform.
template <int STAGE_TOK>
__device__ __forceinline__ bool next_stage(Cursor& c, const int* units, int n_units) {
  c.sb0 += STAGE_TOK;
  while (c.sb0 >= c.vb) {
    if (++c.u >= n_units) return false;
    c.blk = __builtin_amdgcn_readfirstlane(units[2 * c.u]);
    c.vb = __builtin_amdgcn_readfirstlane(units[2 * c.u + 1]);
    c.sb0 = 0;
  }
  return true;
}

// As next_stage for a split without a block table: unit u is block
// first + u * stride and vraw[u] its raw valid count (LDS, copied straight
// from the valid array), clamped here.
template <int STAGE_TOK>
__device__ __forceinline__ bool next_stage_direct(Cursor& c, const int* vraw, int first, int stride,
                                                  int block_tokens, int n_units) {
  c.sb0 += STAGE_TOK;
  while (c.sb0 >= c.vb) {
    if (++c.u >= n_units) return false;
    c.blk = first + c.u * stride;
    c.vb = __builtin_amdgcn_readfirstlane(clamp_valid(vraw[c.u], block_tokens));
    c.sb0 = 0;
  }
  return true;
}

// s_waitcnt immediate waiting until at most n vector-memory operations of
// this wave are outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14)
constexpr int vmcnt_wait(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// ----------------------------------------------------------- query set-up ---
template <int QUADS, int QSPLIT>
struct QueryOps {
  u32x4 qa[QUADS][QSPLIT][4];
  f32x4 qcorr[QUADS];
  float kscale[QUADS];
};

// Query operands of a kv head (gq query heads, QUADS = ceil(gq / 4) groups of
// 4), each value converted once: they are built through LDS scratch of the
// calling wave (coop_scratch_bytes, 16-byte aligned).  Writer lane L = 16h + 4q + m forms
// slot group (m, q) of query head h (of each quad) -- the 8 dims
// qk_dim(m, q, .) -- then every A-operand lane (li, lq) reads its rows back.
// Stores are unconditional, one slot per lane: a store under a lane condition
// to an address other lanes share may be compiled as a read-select-write by
// every lane, and the lanes then race.
template <int QUADS>
constexpr int coop_scratch_bytes = QUADS * 2560;

// The two phases of coop_query: the loads (issued early, so that their
// latency overlaps the first stage's copies) and the build.
template <int QUADS>
struct QueryRaw {
  float x[QUADS][8];  // writer lane's slot group, per quad
};

template <int BITS, int QUADS, typename QT>
__device__ __forceinline__ QueryRaw<QUADS> coop_query_load(const void* query, int gq, int head0, int lane) {
  const int h = lane >> 4, q = (lane >> 2) & 3, m = lane & 3;
  QueryRaw<QUADS> r;
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    const int hq = quad * 4 + h;
    const bool have = hq < gq;
    const int base = (head0 + (have ? hq : 0)) * 128;
    // every load is issued (the head is clamped into range) and masked
    // afterwards: a load under a lane condition becomes a branch with a wait
    // for all outstanding memory operations at its end -- including the stage
    // copies already in flight
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
      const float v = load_query<QT>(query, base + qk_dim<BITS>(m, q, sl));
      r.x[quad][sl] = have ? v : 0.0f;
    }
  }
  return r;
}

template <int BITS, int QUADS, int QSPLIT>
__device__ __forceinline__ void coop_query_build(QueryOps<QUADS, QSPLIT>& qo, const QueryRaw<QUADS>& r,
                                                 float scale_log2, int lane, uint8_t* scratch) {
  const int li = lane & 15, lq = lane >> 4;
  const int h = lane >> 4;
  uint8_t* hi_s = scratch;                                               // [quad][head][q][m] x 16 B
  uint8_t* lo_s = scratch + QUADS * 1024;                                // same, lo parts
  float* corr_s = reinterpret_cast<float*>(scratch + QUADS * 2048);      // [quad][head][lane16]
  float* ksc_s = corr_s + QUADS * 64;                                    // [quad][head][lane16]
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    const float* x = r.x[quad];
    float mx = 0.0f;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) mx = fmaxf(mx, fabsf(x[sl]));
    mx = row_max16(mx);  // over the head's 128 dims
    int ex = 0;
    if (mx > 0.0f && isfinite(mx)) {
      frexpf(mx, &ex);
      ex -= 1;
    }
    _Float16 hi[8], lo[8];
    float part = 0.0f;  // sum over the slot group of (hi + lo) * OFF
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
      const float y = ldexpf(x[sl], -ex) * qk_factor<BITS>(lane & 3, sl);
      hi[sl] = static_cast<_Float16>(y);
      lo[sl] = QSPLIT == 2 ? static_cast<_Float16>(y - static_cast<float>(hi[sl])) : static_cast<_Float16>(0.0f);
      part += (static_cast<float>(hi[sl]) + static_cast<float>(lo[sl])) * qk_off<BITS>(lane & 3, sl);
    }
    const int slot = ((quad * 4 + h) * 16 + (lane & 15)) * 16;
    *reinterpret_cast<u32x4*>(hi_s + slot) =
        u32x4{pack_half2(hi[0], hi[1]), pack_half2(hi[2], hi[3]), pack_half2(hi[4], hi[5]), pack_half2(hi[6], hi[7])};
    if (QSPLIT == 2)
      *reinterpret_cast<u32x4*>(lo_s + slot) =
          u32x4{pack_half2(lo[0], lo[1]), pack_half2(lo[2], lo[3]), pack_half2(lo[4], lo[5]), pack_half2(lo[6], lo[7])};
    // group q = the 4 lanes m = 0..3
    part += __shfl_xor(part, 1, kWave);
    part += __shfl_xor(part, 2, kWave);
    corr_s[(quad * 4 + h) * 16 + (lane & 15)] = part;
    ksc_s[(quad * 4 + h) * 16 + (lane & 15)] = kQkG<BITS> * scale_log2 * exp2f(static_cast<float>(ex));
  }
  // (one wave wrote, the same wave reads: LDS keeps its order)
#pragma unroll
  for (int quad = 0; quad < QUADS; ++quad) {
    // A row (head li/4, group li%4) is non-zero only in lane group lq == li%4
    // (rows of absent heads were written as zeros)
    const bool live = (li & 3) == lq;
    const int row = ((quad * 4 + (li >> 2)) * 16 + 4 * lq) * 16;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(hi_s + row + 16 * mm);
      qo.qa[quad][0][mm] = live ? v : u32x4{0u, 0u, 0u, 0u};
      if (QSPLIT == 2) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(lo_s + row + 16 * mm);
        qo.qa[quad][QSPLIT - 1][mm] = live ? w : u32x4{0u, 0u, 0u, 0u};
      }
    }
    // C init of QK lane (li, lq), register g: row (head lq, group g), the sum
    // held by lane 4g of the writer row
#pragma unroll
    for (int g = 0; g < 4; ++g) qo.qcorr[quad][g] = -corr_s[(quad * 4 + lq) * 16 + 4 * g];
    qo.kscale[quad] = ksc_s[(quad * 4 + lq) * 16];
  }
}

template <int BITS, int QUADS, int QSPLIT, typename QT>
__device__ __forceinline__ void coop_query(QueryOps<QUADS, QSPLIT>& qo, const void* query, int gq, float scale_log2,
                                           int head0, int lane, uint8_t* scratch) {
  coop_query_build<BITS, QUADS, QSPLIT>(qo, coop_query_load<BITS, QUADS, QT>(query, gq, head0, lane), scale_log2,
                                        lane, scratch);
}


}  // namespace
}  // namespace kvssd
