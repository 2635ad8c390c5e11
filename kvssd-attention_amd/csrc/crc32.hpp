// CRC-32 on the GPU, shared by the v1 record codec (records.hip) and the
// vLLM block codec (vllm_codec.hip).
//
// CRC-32 is zlib's: reflected polynomial 0xEDB88320, register preset to all
// ones, output complemented.  Polynomials over GF(2) are held bit-reflected
// (bit 31 is the coefficient of x^0).  The raw register update (preset 0, no
// complement) is linear: crc_raw(A || B) = x^(8|B|) crc_raw(A) + crc_raw(B)
// (mod P), and leading zero bytes do not change crc_raw, so a payload is
// virtually left-padded with zeros to a whole number of pieces.  Finally
// crc32(D) = x^(8|D|) * 0xFFFFFFFF + crc_raw(D) + 0xFFFFFFFF.
//
// Chunked form (layouts whose four payload arrays are 16-byte multiples, the
// usual case): a workgroup of 1024 threads covers a record in 16-byte chunks,
// chunk c = j * 1024 + t belonging to thread t.  Every thread issues all its
// loads at once (coalesced), stores each chunk to its PackedBatch array and
// takes the chunk's crc_raw from the registers with 16 independent table
// lookups (slicing-by-16).  Its own chunks fold by Horner's rule with a
// table-driven multiply by x^(8 * 16384); the 1024 thread values then fold
// pairwise in 10 levels (x^(8 * 16 * 2^k)).  Other layouts take the general
// form: 1024 contiguous segments through a slicing-by-4 walk, then the same
// 10-level fold.  All tables are built at compile time.
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

namespace kvssd {
namespace {

constexpr uint32_t kPoly = 0xEDB88320u;
constexpr int kCrcThreads = 1024;          // segments per record
constexpr int kCrcLevels = 10;             // log2(kCrcThreads)

// a * b mod P (reflected representation)
__host__ __device__ constexpr uint32_t gf_mul(uint32_t a, uint32_t b) {
  uint32_t p = 0;
  for (int i = 0; i < 32; ++i) {
    if (a & (0x80000000u >> i)) p ^= b;
    b = (b & 1u) ? (b >> 1) ^ kPoly : b >> 1;  // b *= x
  }
  return p;
}

// x^(8 n) mod P
__host__ __device__ constexpr uint32_t x_pow_bytes(uint64_t n) {
  uint32_t r = 0x80000000u;   // x^0
  uint32_t sq = 0x00800000u;  // x^8
  while (n) {
    if (n & 1u) r = gf_mul(r, sq);
    sq = gf_mul(sq, sq);
    n >>= 1;
  }
  return r;
}

constexpr int kChunkBytes = 16;
constexpr int kStrideBytes = kChunkBytes * kCrcThreads;  // one row of chunks
constexpr int kMaxRows = 16;                             // chunked form: payload <= 256 KiB

// slice[k][n]: raw register after byte n followed by k zero bytes;
// horner[k][b]: x^(8 * kStrideBytes) * (b << 8k), so that the product with any
// word is the XOR of four lookups
struct CrcTables {
  uint32_t slice[16][256];
  uint32_t horner[4][256];
};

constexpr CrcTables make_crc_tables() {
  CrcTables t{};
  for (uint32_t n = 0; n < 256; ++n) {
    uint32_t c = n;
    for (int i = 0; i < 8; ++i) c = (c & 1u) ? (c >> 1) ^ kPoly : c >> 1;
    t.slice[0][n] = c;
  }
  for (int k = 1; k < 16; ++k)
    for (uint32_t n = 0; n < 256; ++n) {
      const uint32_t c = t.slice[k - 1][n];
      t.slice[k][n] = t.slice[0][c & 0xFFu] ^ (c >> 8);  // one more zero byte
    }
  const uint32_t m = x_pow_bytes(kStrideBytes);
  for (int k = 0; k < 4; ++k)
    for (uint32_t b = 0; b < 256; ++b) t.horner[k][b] = gf_mul(m, b << (8 * k));
  return t;
}

__device__ const CrcTables kCrcTables = make_crc_tables();

// Position multipliers of the chunked form: chunk[t] = x^(8 * 16 * (1023 - t)),
// row[t] = x^(8 * 16384 * (1023 - t)) -- the shift of piece t of 1024 equal
// pieces to the end of the message they form.
struct PosTables {
  uint32_t chunk[kCrcThreads];
  uint32_t row[kCrcThreads];
};

constexpr PosTables make_pos_tables() {
  PosTables p{};
  const uint32_t sc = x_pow_bytes(16), sr = x_pow_bytes(16384);
  p.chunk[kCrcThreads - 1] = 0x80000000u;  // x^0
  p.row[kCrcThreads - 1] = 0x80000000u;
  for (int t = kCrcThreads - 1; t > 0; --t) {
    p.chunk[t - 1] = gf_mul(p.chunk[t], sc);
    p.row[t - 1] = gf_mul(p.row[t], sr);
  }
  return p;
}

__device__ const PosTables kPosTables = make_pos_tables();

// a * b mod P without branches (device)
__device__ __forceinline__ uint32_t gf_mul_dev(uint32_t a, uint32_t b) {
  uint32_t p = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    p ^= b & (0u - ((a >> (31 - i)) & 1u));
    b = (b >> 1) ^ (kPoly & (0u - (b & 1u)));
  }
  return p;
}

// raw register after byte n followed by k zero bytes (slicing-by-4 table k)
__device__ __forceinline__ uint32_t crc_table_entry(int k, uint32_t n) { return kCrcTables.slice[k][n]; }

struct CrcPlan {
  uint32_t seg_bytes;           // L: bytes per segment (multiple of 4)
  uint32_t pad;                 // virtual leading zero bytes
  uint32_t len;                 // payload bytes covered
  uint32_t x_len;               // x^(8 len) mod P
  uint32_t level[kCrcLevels];   // x^(8 L 2^k) mod P
};

CrcPlan make_crc_plan(uint32_t len) {
  CrcPlan c{};
  const uint32_t per = (len + kCrcThreads - 1) / kCrcThreads;
  c.seg_bytes = (per + 3u) & ~3u;
  c.pad = c.seg_bytes * kCrcThreads - len;
  c.len = len;
  c.x_len = x_pow_bytes(len);
  for (int k = 0; k < kCrcLevels; ++k) c.level[k] = x_pow_bytes(static_cast<uint64_t>(c.seg_bytes) << k);
  return c;
}

// zlib CRC-32 of data[0 .. plan.len), data 4-byte aligned; every thread of a
// kCrcThreads workgroup calls it; tab = the four slicing tables in LDS,
// seg = kCrcThreads words of LDS.  Returns the CRC in every thread.
__device__ uint32_t block_crc32(const uint8_t* data, const CrcPlan& plan, const uint32_t (*tab)[256], uint32_t* seg) {
  const int tid = threadIdx.x;
  const int64_t v0 = static_cast<int64_t>(tid) * plan.seg_bytes - plan.pad;  // first real byte of the segment
  uint32_t crc = 0;
  if ((plan.len & 3u) == 0) {
    // pad is then a multiple of 4: whole dwords, real or virtual zeros
    for (uint32_t i = 0; i < plan.seg_bytes; i += 4) {
      const int64_t at = v0 + i;
      if (at < 0) continue;  // leading zeros keep the raw register at 0
      crc ^= *reinterpret_cast<const uint32_t*>(data + at);
      crc = tab[3][crc & 0xFFu] ^ tab[2][(crc >> 8) & 0xFFu] ^ tab[1][(crc >> 16) & 0xFFu] ^ tab[0][crc >> 24];
    }
  } else {
    for (uint32_t i = 0; i < plan.seg_bytes; ++i) {
      const int64_t at = v0 + i;
      if (at < 0) continue;
      crc = tab[0][(crc ^ data[at]) & 0xFFu] ^ (crc >> 8);
    }
  }
  seg[tid] = crc;
  for (int k = 0; k < kCrcLevels; ++k) {
    __syncthreads();
    const int span = 1 << k;
    if ((tid & (2 * span - 1)) == 0) seg[tid] = gf_mul(plan.level[k], seg[tid]) ^ seg[tid + span];
  }
  __syncthreads();
  const uint32_t raw = seg[0];
  __syncthreads();  // seg may be reused by the caller
  return gf_mul(plan.x_len, 0xFFFFFFFFu) ^ raw ^ 0xFFFFFFFFu;
}

__device__ __forceinline__ void fill_crc_tables(uint32_t (*tab)[256]) {
  for (int i = threadIdx.x; i < 4 * 256; i += blockDim.x) tab[i >> 8][i & 255] = crc_table_entry(i >> 8, i & 255);
}

// ----------------------------------------------------------- chunked form ---
struct ChunkLds {
  uint32_t slice[16][256];
  uint32_t horner[4][256];
  uint32_t seg[kCrcThreads];
};

__device__ __forceinline__ void load_chunk_tables(ChunkLds& l) {
  const uint32_t* src = &kCrcTables.slice[0][0];
  uint32_t* dst = &l.slice[0][0];
  uint32_t v[5];
#pragma unroll
  for (int j = 0; j < 5; ++j) v[j] = src[threadIdx.x + j * kCrcThreads];  // slice then horner
#pragma unroll
  for (int j = 0; j < 5; ++j) dst[threadIdx.x + j * kCrcThreads] = v[j];
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes at a 4-byte aligned address
__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
  u32x4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 4), 16);
  return v;
}

__device__ __forceinline__ uint32_t crc16_raw(const ChunkLds& l, u32x4 v) {
  uint32_t c = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t x = v[w];
#pragma unroll
    for (int b = 0; b < 4; ++b) c ^= l.slice[15 - 4 * w - b][(x >> (8 * b)) & 0xFFu];
  }
  return c;
}

__device__ __forceinline__ uint32_t mul_stride(const ChunkLds& l, uint32_t a) {
  return l.horner[0][a & 0xFFu] ^ l.horner[1][(a >> 8) & 0xFFu] ^ l.horner[2][(a >> 16) & 0xFFu] ^
         l.horner[3][a >> 24];
}

// Chunk geometry of a payload of `len` bytes (a multiple of 16): `rows` rows of
// 1024 chunks, the first `pad` bytes virtual zeros.
struct ChunkPlan {
  int rows;
  int64_t pad;
  uint32_t x_len;  // x^(8 len) mod P
};

ChunkPlan make_chunk_plan(uint32_t len) {
  ChunkPlan c{};
  c.rows = static_cast<int>((len + kStrideBytes - 1) / kStrideBytes);
  c.pad = static_cast<int64_t>(c.rows) * kStrideBytes - len;
  c.x_len = x_pow_bytes(len);
  return c;
}

// byte offset (into the payload) of chunk row j of this thread; negative = virtual zeros
__device__ __forceinline__ int64_t chunk_offset(const ChunkPlan& c, int j) {
  return (static_cast<int64_t>(j) * kCrcThreads + threadIdx.x) * kChunkBytes - c.pad;
}

// Fold the 1024 per-thread raw values h, thread t's piece followed by the
// pieces of threads t+1 .. 1023 (pos[t] = the shift of piece t to the end):
// one multiply per thread, then an XOR reduction.  The raw register value of
// the whole message is returned in every thread.
__device__ uint32_t fold_pos(ChunkLds& l, const uint32_t* pos, uint32_t h) {
  const int tid = threadIdx.x;
  uint32_t v = gf_mul_dev(pos[tid], h);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64));
  if ((tid & 63) == 0) l.seg[tid >> 6] = v;
  __syncthreads();
  uint32_t raw = 0;
#pragma unroll
  for (int w = 0; w < kCrcThreads / 64; ++w) raw ^= l.seg[w];
  __syncthreads();  // seg may be reused by the caller
  return raw;
}

// zlib's CRC-32 of a message of x_len = x^(8 len) from its raw register value
__host__ __device__ inline uint32_t crc_from_raw(uint32_t x_len, uint32_t raw) {
  return gf_mul(x_len, 0xFFFFFFFFu) ^ raw ^ 0xFFFFFFFFu;
}

// Fold this thread's Horner value `h` (its 16-byte chunks) with every other
// thread's: the payload's zlib CRC-32, returned in every thread.
__device__ uint32_t fold_chunks(ChunkLds& l, const ChunkPlan& c, uint32_t h) {
  return crc_from_raw(c.x_len, fold_pos(l, kPosTables.chunk, h));
}

}  // namespace
}  // namespace kvssd
