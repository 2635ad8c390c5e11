/*
 * CPU oracle for the fused INT2/INT4 dequant + decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is a plain-C restatement of the
 * reference algorithm, used to check results by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  Nothing in the
 * kvssd package links, loads or calls it; the product path never routes
 * through it.
 *
 * Each function names the reference file:line it restates.  Accumulation is
 * done in double precision so the oracle is at least as accurate as the
 * reference's fp32 torch computation; the fp32 dequantised values themselves
 * are exact (code <= 4 bits times an fp16 scale fits a float).
 *
 * Parity pins (tests/test_oracle.py):
 *   orc_f32_to_f16 / orc_f16_to_f32  numpy float16 casts over all 65536 halves
 *                                    and a dense float sweep
 *   orc_quantize_groups              closed-form known answers (half-even,
 *                                    all-zero group, INT2 group) + invariants
 *   orc_pack_codes / orc_unpack_codes  known answers + exhaustive 256-byte sweep
 *   orc_decode_attention             torch float64 scaled_dot_product_attention,
 *                                    single-token / equal-key closed forms,
 *                                    pure-Python brute force on tiny inputs
 *   orc_merge                        split-anywhere invariant vs one call
 *   orc_crc32                        zlib.crc32 and crc32("123456789")
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------- fp16 --- */

/* IEEE binary16 -> binary32 (exact).  The reference stores scales as fp16
 * (src/kvssd/quant.py:61) and reads them with .float() (quant.py:72,
 * backends/reference.py:31). */
ORC_API float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float v = (float)man * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

/* binary32 -> binary16 with round-to-nearest-even, subnormals kept, overflow to
 * infinity: the semantics of torch's .to(torch.float16) used for the scales
 * (src/kvssd/quant.py:61). */
ORC_API uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) { /* inf or nan */
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    return (uint16_t)(sign | 0x7C00u);
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal */
    if (ax < 0x33000000u) return sign;                        /* < 2^-25 rounds to 0 */
    /* value = m * 2^(e-150); the half subnormal unit is 2^-24, so the result
     * mantissa is round(m * 2^(e-126)) = round(m >> (126 - e)), 14 <= shift <= 24.
     * A carry to 0x400 lands exactly on the smallest normal half. */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    int shift = 126 - (int)e;
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (ax >> 23) - 112u;
  uint32_t m = ax & 0x7FFFFFu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1; /* may carry into exp */
  return (uint16_t)(sign | q);
}

/* --------------------------------------------------------- quantisation --- */

/* Symmetric groupwise quantiser, restating src/kvssd/quant.py:49-65 in fp32:
 *   scale32 = max(|x|).clamp_min(1e-8) / (2^(bits-1)-1)       (quant.py:56)
 *   code    = clamp(round_half_even(x / scale32), -mid, pmax) + mid (quant.py:57-58)
 *   scale   = fp16(scale32)                                   (quant.py:61)
 * x holds n_groups * group_size floats; codes one byte per element. */
ORC_API void orc_quantize_groups(const float* x, int64_t n_groups, int group_size, int bits,
                                 uint8_t* codes, uint16_t* scales) {
  const int mid = 1 << (bits - 1);
  const float pmax = (float)(mid - 1);
  for (int64_t gi = 0; gi < n_groups; ++gi) {
    const float* gx = x + gi * group_size;
    float amax = 0.0f;
    for (int i = 0; i < group_size; ++i) {
      float a = fabsf(gx[i]);
      if (a > amax || isnan(a)) amax = a;
    }
    float clamped = amax < 1e-8f ? 1e-8f : amax;
    volatile float scale32 = clamped / pmax; /* IEEE fp32 division, as torch */
    for (int i = 0; i < group_size; ++i) {
      volatile float ratio = gx[i] / scale32;
      float r = nearbyintf(ratio); /* default rounding mode: half to even */
      if (r < (float)-mid) r = (float)-mid;
      if (r > pmax) r = pmax;
      codes[gi * group_size + i] = (uint8_t)(int)(r + (float)mid);
    }
    scales[gi] = orc_f32_to_f16(scale32);
  }
}

/* Low-bits-first packing along the last dim: src/kvssd/quant.py:28-37. */
ORC_API void orc_pack_codes(const uint8_t* codes, int64_t n_codes, int bits, uint8_t* packed) {
  const int per = 8 / bits;
  for (int64_t b = 0; b < n_codes / per; ++b) {
    unsigned v = 0;
    for (int i = 0; i < per; ++i) v |= (unsigned)(codes[b * per + i] & ((1u << bits) - 1u)) << (i * bits);
    packed[b] = (uint8_t)v;
  }
}

/* Inverse of orc_pack_codes, as unpack_codes: src/kvssd/quant.py:40-46. */
ORC_API void orc_unpack_codes(const uint8_t* packed, int64_t n_bytes, int bits, uint8_t* codes) {
  const int per = 8 / bits;
  for (int64_t b = 0; b < n_bytes; ++b)
    for (int i = 0; i < per; ++i) codes[b * per + i] = (uint8_t)((packed[b] >> (i * bits)) & ((1u << bits) - 1u));
}

/* Element (blk, t, h, d) of a packed [NB, BT, KVH, PD] tensor with fp16 scales
 * [NB, BT, KVH, G]: ((code - mid) * scale) as in backends/reference.py:29-32 and
 * csrc/fused_decode.cu:50-56.  Exact in fp32 and in double. */
static inline double dequant(const uint8_t* packed, const uint16_t* scales, int64_t row, int pd, int groups,
                             int d, int bits, int g) {
  const int per = 8 / bits;
  const unsigned byte = packed[row * pd + d / per];
  const int code = (int)((byte >> ((d % per) * bits)) & ((1u << bits) - 1u));
  const int mid = 1 << (bits - 1);
  return (double)(code - mid) * (double)orc_f16_to_f32(scales[row * groups + d / g]);
}

/* Rows of a block that take part for its count v: the rows Python's slice
 * keys[index, :v] keeps in src/kvssd/backends/reference.py:38-40, i.e.
 * min(v, BT) for v >= 0 and max(BT + v, 0) for v < 0. */
static inline int slice_rows(int v, int bt) {
  const int n = v < 0 ? bt + v : v;
  return n < 0 ? 0 : (n > bt ? bt : n);
}

/* Decode attention over a packed batch: restates
 * ReferenceAttentionBackend.run (src/kvssd/backends/reference.py:22-50).
 *   - tokens are the rows keys[b, :valid[b]] of each block (slice_rows), blocks
 *     in batch order (reference.py:36-42);
 *   - GQA map qh -> qh / (QH/KVH) (reference.py:45);
 *   - s = sm_scale * q.k, lse = logsumexp(s), out = softmax(s) @ V
 *     (reference.py:46-49).
 * block_table (n_sel entries) selects blocks of the packed arrays; NULL means
 * blocks 0..NB-1 in order.  q is fp32 [QH, D]; out fp32 [QH, D]; lse fp32 [QH].
 * With no valid token at all the result is out = 0, lse = -inf, which is what
 * reference.py:46-49 returns for an empty token set.
 * Returns 0, or -1 on an invalid shape. */
ORC_API int orc_decode_attention(int qh, int kvh, int d, int nb, int bt, int bits, int g, const float* q,
                                 const uint8_t* pk, const uint8_t* pv, const uint16_t* sk, const uint16_t* sv,
                                 const int32_t* valid, const int32_t* block_table, int n_sel, double sm_scale,
                                 float* out, float* lse, int threads) {
  if (qh <= 0 || kvh <= 0 || qh % kvh || d <= 0 || g <= 0 || d % g || (bits != 2 && bits != 4)) return -1;
  const int pd = d * bits / 8;
  const int groups = d / g;
  const int gq = qh / kvh;
  const int nsel = block_table ? n_sel : nb;
  int64_t total = 0;
  for (int i = 0; i < nsel; ++i) {
    int b = block_table ? block_table[i] : i;
    if (b < 0 || b >= nb) return -1;
    total += slice_rows(valid[b], bt);
  }
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel for schedule(dynamic, 1)
  for (int h = 0; h < qh; ++h) {
    const int kv = h / gq;
    double* scores = (double*)malloc(sizeof(double) * (size_t)(total > 0 ? total : 1));
    double* acc = (double*)calloc((size_t)d, sizeof(double));
    double mx = -INFINITY;
    int64_t n = 0;
    for (int i = 0; i < nsel; ++i) {
      int b = block_table ? block_table[i] : i;
      const int v = slice_rows(valid[b], bt);
      for (int t = 0; t < v; ++t) {
        int64_t row = ((int64_t)b * bt + t) * kvh + kv;
        double s = 0.0;
        for (int e = 0; e < d; ++e) s += (double)q[h * d + e] * dequant(pk, sk, row, pd, groups, e, bits, g);
        s *= sm_scale;
        scores[n++] = s;
        if (s > mx) mx = s;
      }
    }
    double sum = 0.0;
    n = 0;
    for (int i = 0; i < nsel; ++i) {
      int b = block_table ? block_table[i] : i;
      const int v = slice_rows(valid[b], bt);
      for (int t = 0; t < v; ++t) {
        int64_t row = ((int64_t)b * bt + t) * kvh + kv;
        double p = exp(scores[n++] - mx);
        sum += p;
        for (int e = 0; e < d; ++e) acc[e] += p * dequant(pv, sv, row, pd, groups, e, bits, g);
      }
    }
    for (int e = 0; e < d; ++e) out[h * d + e] = sum > 0.0 ? (float)(acc[e] / sum) : 0.0f;
    lse[h] = sum > 0.0 ? (float)(mx + log(sum)) : -INFINITY;
    free(scores);
    free(acc);
  }
  return 0;
}

/* Exact merge of two normalised chunks: src/kvssd/attention.py:91-102
 *   L = logaddexp(La, Lb); O = Oa e^(La-L) + Ob e^(Lb-L).
 * A chunk with L = -inf (no tokens) contributes nothing; two empty chunks give
 * O = 0, L = -inf (the result of attending over their empty union). */
ORC_API void orc_merge(int rows, int d, const float* oa, const float* la, const float* ob, const float* lb,
                       float* out, float* lout) {
  for (int r = 0; r < rows; ++r) {
    double a = la[r], b = lb[r];
    double m = a > b ? a : b;
    if (m == -INFINITY) {
      for (int e = 0; e < d; ++e) out[r * d + e] = 0.0f;
      lout[r] = -INFINITY;
      continue;
    }
    double wa = exp(a - m), wb = exp(b - m);
    double l = m + log(wa + wb);
    wa = exp(a - l);
    wb = exp(b - l);
    for (int e = 0; e < d; ++e) out[r * d + e] = (float)(wa * oa[r * d + e] + wb * ob[r * d + e]);
    lout[r] = (float)l;
  }
}

/* ------------------------------------------------------------------ crc --- */

/* Reflected CRC-32 (polynomial 0xEDB88320), the checksum zlib.crc32 computes
 * over each record payload (src/kvssd/format.py:115, :151). */
ORC_API uint32_t orc_crc32(const uint8_t* data, size_t n, uint32_t crc) {
  static uint32_t table[256];
  static int ready = 0;
  if (!ready) {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
      table[i] = c;
    }
    ready = 1;
  }
  crc = ~crc;
  for (size_t i = 0; i < n; ++i) crc = table[(crc ^ data[i]) & 0xFFu] ^ (crc >> 8);
  return ~crc;
}
