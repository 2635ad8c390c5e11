// GPU codec of the v1 KV block record (src/kvssd/format.py:14-177):
//
// * gather: raw records (as read from the store, copied to HBM in one span)
//   -> the PackedBatch arrays, with decode_record's header, layout and
//   payload CRC-32 checks (format.py:134-177); replaces the loader's per-block
//   payload clones and the pipeline's per-array stacking
//   (src/kvssd/loader.py:73-91, src/kvssd/pipeline.py:98-108);
// * quantize: bit-exact twin of quantize_tensor (src/kvssd/quant.py:49-65);
// * encode: KVCacheStore.create's block loop for one layer (zero-padded last
//   block, src/kvssd/store.py:46-63) -- quantise keys and values and write
//   whole records with their CRC-32 (encode_record, format.py:104-131); one
//   fused kernel for the common layouts, else a payload and a header pass.
//
// CRC-32 machinery (zlib's CRC, chunked and general forms): crc32.hpp.
#include "crc32.hpp"
#include "decode.hpp"

namespace kvssd {
namespace {

constexpr int kHeaderBytes = 52;      // "<8sIIIIIIIIIII"
constexpr int kRecordAlign = 4096;
constexpr uint32_t kMagic0 = 0x5353564Bu;  // "KVSS", little-endian
constexpr uint32_t kMagic1 = 0x31303044u;  // "D001"

// bytes [0, len) from src to dst, dwords when both ends allow
__device__ __forceinline__ void copy_region(const uint8_t* src, uint8_t* dst, int64_t len) {
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | static_cast<uintptr_t>(len)) & 3u) == 0) {
    const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
    for (int64_t i = threadIdx.x; i < len / 4; i += blockDim.x) d[i] = s[i];
  } else {
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) dst[i] = src[i];
  }
}

struct Layout {
  int bits, block_tokens, kv_heads, head_dim, group_size;
  __host__ __device__ int64_t scale_bytes() const { return static_cast<int64_t>(block_tokens) * kv_heads * (head_dim / group_size) * 2; }
  __host__ __device__ int64_t packed_bytes() const { return static_cast<int64_t>(block_tokens) * kv_heads * head_dim * bits / 8; }
  __host__ __device__ int64_t payload_bytes() const { return 2 * scale_bytes() + 2 * packed_bytes(); }
  __host__ __device__ int64_t record_bytes() const {
    const int64_t n = kHeaderBytes + payload_bytes();
    return (n + kRecordAlign - 1) / kRecordAlign * kRecordAlign;
  }
};

// ------------------------------------------------------------------ gather ---
struct GatherParams {
  const uint8_t* records;
  int64_t stride;
  int n, verify;
  Layout lay;
  CrcPlan plan;
  uint8_t *pk, *pv, *sk, *sv;
  int32_t* valid;
  int32_t* status;
};

// one workgroup per record; status: 0 ok, 1 invalid header (magic / version),
// 2 layout differs from the expected one, 3 payload length or CRC mismatch
__global__ __launch_bounds__(kCrcThreads) void gather_records_kernel(GatherParams p) {
  __shared__ uint32_t tab[4][256];
  __shared__ uint32_t seg[kCrcThreads];
  __shared__ uint32_t hdr[kHeaderBytes / 4];
  const int r = blockIdx.x;
  const uint8_t* rec = p.records + static_cast<int64_t>(r) * p.stride;
  fill_crc_tables(tab);
  if (threadIdx.x < kHeaderBytes / 4) hdr[threadIdx.x] = reinterpret_cast<const uint32_t*>(rec)[threadIdx.x];
  __syncthreads();
  int status = 0;
  if (hdr[0] != kMagic0 || hdr[1] != kMagic1 || hdr[2] != 1u) {
    status = 1;
  } else if (hdr[6] != static_cast<uint32_t>(p.lay.bits) || hdr[7] != static_cast<uint32_t>(p.lay.block_tokens) ||
             hdr[8] != static_cast<uint32_t>(p.lay.kv_heads) || hdr[9] != static_cast<uint32_t>(p.lay.head_dim) ||
             hdr[10] != static_cast<uint32_t>(p.lay.group_size)) {
    status = 2;
  }
  const int64_t s = p.lay.scale_bytes(), pb = p.lay.packed_bytes();
  const uint8_t* pay = rec + kHeaderBytes;
  copy_region(pay, p.sk + r * s, s);
  copy_region(pay + s, p.sv + r * s, s);
  copy_region(pay + 2 * s, p.pk + r * pb, pb);
  copy_region(pay + 2 * s + pb, p.pv + r * pb, pb);
  if (p.verify && status == 0) {
    // a record written for this layout has exactly the layout's payload
    if (hdr[11] != p.plan.len) {
      status = 3;
    } else {
      const uint32_t crc = block_crc32(pay, p.plan, tab, seg);
      if (crc != hdr[12]) status = 3;
    }
  }
  if (threadIdx.x == 0) {
    p.status[r] = status;
    p.valid[r] = static_cast<int32_t>(hdr[5]);
  }
}

// chunked form of gather_records_kernel (same statuses), for layouts whose
// four arrays are 16-byte multiples and 16-byte aligned destinations
__global__ __launch_bounds__(kCrcThreads) void gather_chunked_kernel(GatherParams p, ChunkPlan c) {
  __shared__ ChunkLds lds;
  __shared__ uint32_t hdr[kHeaderBytes / 4];
  const int r = blockIdx.x;
  const uint8_t* rec = p.records + static_cast<int64_t>(r) * p.stride;
  const uint8_t* pay = rec + kHeaderBytes;
  u32x4 v[kMaxRows];
#pragma unroll
  for (int j = 0; j < kMaxRows; ++j) {
    v[j] = u32x4{0u, 0u, 0u, 0u};
    if (j < c.rows) {
      const int64_t o = chunk_offset(c, j);
      if (o >= 0) v[j] = load16(pay + o);
    }
  }
  if (threadIdx.x < kHeaderBytes / 4) hdr[threadIdx.x] = reinterpret_cast<const uint32_t*>(rec)[threadIdx.x];
  if (p.verify) load_chunk_tables(lds);
  const int64_t sb = p.lay.scale_bytes(), pb = p.lay.packed_bytes();
#pragma unroll
  for (int j = 0; j < kMaxRows; ++j) {
    if (j < c.rows) {
      const int64_t o = chunk_offset(c, j);
      if (o >= 0) {
        uint8_t* dst;
        if (o < sb) dst = p.sk + r * sb + o;
        else if (o < 2 * sb) dst = p.sv + r * sb + (o - sb);
        else if (o < 2 * sb + pb) dst = p.pk + r * pb + (o - 2 * sb);
        else dst = p.pv + r * pb + (o - 2 * sb - pb);
        *reinterpret_cast<u32x4*>(dst) = v[j];
      }
    }
  }
  __syncthreads();
  int status = 0;
  if (hdr[0] != kMagic0 || hdr[1] != kMagic1 || hdr[2] != 1u) {
    status = 1;
  } else if (hdr[6] != static_cast<uint32_t>(p.lay.bits) || hdr[7] != static_cast<uint32_t>(p.lay.block_tokens) ||
             hdr[8] != static_cast<uint32_t>(p.lay.kv_heads) || hdr[9] != static_cast<uint32_t>(p.lay.head_dim) ||
             hdr[10] != static_cast<uint32_t>(p.lay.group_size)) {
    status = 2;
  }
  // status, p.verify and the header are the same in every thread, so the
  // fold's barriers are reached by the whole workgroup or by none of it
  if (p.verify && status == 0) {
    if (hdr[11] != p.plan.len) {
      status = 3;
    } else {
      uint32_t h = 0;
#pragma unroll
      for (int j = 0; j < kMaxRows; ++j)
        if (j < c.rows) h = mul_stride(lds, h) ^ crc16_raw(lds, v[j]);
      if (fold_chunks(lds, c, h) != hdr[12]) status = 3;
    }
  }
  if (threadIdx.x == 0) {
    p.status[r] = status;
    p.valid[r] = static_cast<int32_t>(hdr[5]);
  }
}

// ---------------------------------------------------------------- quantize ---
template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) {  // bfloat16 bits
  return __builtin_bit_cast(float, static_cast<uint32_t>(v) << 16);
}

// one group (group_size consecutive values) -> packed bytes + fp16 scale, as
// quantize_tensor: scale32 = max|x| (at least 1e-8) / (2^(bits-1) - 1) with
// IEEE division, code = clamp(rint(x / scale32), -mid, mid - 1) + mid, codes
// packed low bits first, scale stored as fp16 (round to nearest even).  A
// null src reads zeros (padding tokens).
template <typename T>
__device__ __forceinline__ void quantize_group(const T* src, int group_size, int bits, uint8_t* packed, uint16_t* scale) {
  float amax = 0.0f;
  for (int i = 0; i < group_size; ++i) amax = fmaxf(amax, fabsf(src ? to_f32(src[i]) : 0.0f));
  const int mid = 1 << (bits - 1);
  const float s32 = fmaxf(amax, 1e-8f) / static_cast<float>(mid - 1);
  const int per = 8 / bits;
  for (int b = 0; b < group_size / per; ++b) {
    uint32_t byte = 0;
    for (int j = 0; j < per; ++j) {
      const float x = src ? to_f32(src[b * per + j]) : 0.0f;
      const float c = fminf(fmaxf(rintf(x / s32), static_cast<float>(-mid)), static_cast<float>(mid - 1));
      byte |= static_cast<uint32_t>(static_cast<int>(c) + mid) << (j * bits);
    }
    packed[b] = static_cast<uint8_t>(byte);
  }
  *scale = __builtin_bit_cast(uint16_t, static_cast<_Float16>(s32));
}

// The same arithmetic for a 32-value group held in registers: the group is
// read once with wide loads (src 16-byte aligned) and its packed bytes go out
// in one 4-byte aligned store of 4 (INT4) or 2 (INT2) words.
constexpr int kRegGroup = 32;

template <int BITS>
struct GroupWords {
  uint32_t w[kRegGroup * BITS / 32];  // packed codes, low bits first
  uint16_t scale;                     // fp16 bits
};

template <typename T, int BITS>
__device__ __forceinline__ GroupWords<BITS> quantize_group_words(const T* src) {
  float x[kRegGroup];
  if (src) {
    T v[kRegGroup];
    __builtin_memcpy(v, __builtin_assume_aligned(src, 16), sizeof(v));
#pragma unroll
    for (int i = 0; i < kRegGroup; ++i) x[i] = to_f32(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < kRegGroup; ++i) x[i] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kRegGroup; ++i) amax = fmaxf(amax, fabsf(x[i]));
  constexpr int mid = 1 << (BITS - 1);
  const float s32 = fmaxf(amax, 1e-8f) / static_cast<float>(mid - 1);
  GroupWords<BITS> g;
#pragma unroll
  for (int k = 0; k < kRegGroup * BITS / 32; ++k) g.w[k] = 0;
#pragma unroll
  for (int i = 0; i < kRegGroup; ++i) {
    const float c = fminf(fmaxf(rintf(x[i] / s32), static_cast<float>(-mid)), static_cast<float>(mid - 1));
    g.w[(i * BITS) >> 5] |= static_cast<uint32_t>(static_cast<int>(c) + mid) << ((i * BITS) & 31);
  }
  g.scale = __builtin_bit_cast(uint16_t, static_cast<_Float16>(s32));
  return g;
}

template <typename T, int BITS>
__device__ __forceinline__ void quantize_group_reg(const T* src, uint8_t* packed, uint16_t* scale) {
  const GroupWords<BITS> g = quantize_group_words<T, BITS>(src);
  __builtin_memcpy(__builtin_assume_aligned(packed, 4), g.w, sizeof(g.w));
  *scale = g.scale;
}

// BITS == 0: any group size (quantize_group); BITS == 2 / 4: group_size 32
// in registers (quantize_group_reg)
template <typename T, int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(const T* __restrict__ x, int64_t groups, int group_size, int bits,
                                                       uint8_t* __restrict__ packed, uint16_t* __restrict__ scales) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= groups) return;
  if constexpr (BITS == 0) {
    quantize_group(x + g * group_size, group_size, bits, packed + g * (group_size * bits / 8), scales + g);
  } else {
    quantize_group_reg<T, BITS>(x + g * kRegGroup, packed + g * (kRegGroup * BITS / 8), scales + g);
  }
}

// ------------------------------------------------------------------ encode ---
struct EncodeParams {
  const void* keys;
  const void* values;
  int64_t tokens;
  int n, layer, first_block;
  Layout lay;
  CrcPlan plan;
  uint8_t* records;
  uint32_t* crcs;
};

// phase 1: every (record, key/value, token, kv head, group) quantised into
// the record's payload; tokens past the end read as zeros.  BITS as in
// quantize_kernel.
template <typename T, int BITS>
__global__ __launch_bounds__(256) void encode_payload_kernel(EncodeParams p) {
  const Layout& L = p.lay;
  const int G = L.head_dim / L.group_size;
  const int64_t per_record = static_cast<int64_t>(L.block_tokens) * L.kv_heads * G;  // groups per array
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= 2 * per_record * p.n) return;
  const int r = static_cast<int>(g / (2 * per_record));
  const int64_t rest = g % (2 * per_record);
  const bool is_v = rest >= per_record;
  const int64_t q = is_v ? rest - per_record : rest;  // (token, head, group) within the block
  const int64_t row = q / G;                          // token * kv_heads + head
  const int gi = static_cast<int>(q % G);
  const int64_t token = static_cast<int64_t>(r) * L.block_tokens + row / L.kv_heads;
  const T* base = static_cast<const T*>(is_v ? p.values : p.keys);
  const T* src = token < p.tokens ? base + (token * L.kv_heads + row % L.kv_heads) * L.head_dim + gi * L.group_size
                                  : nullptr;
  uint8_t* pay = p.records + static_cast<int64_t>(r) * L.record_bytes() + kHeaderBytes;
  const int64_t s = L.scale_bytes(), pb = L.packed_bytes();
  uint16_t* scale = reinterpret_cast<uint16_t*>(pay + (is_v ? s : 0)) + q;
  uint8_t* packed = pay + 2 * s + (is_v ? pb : 0) + q * (L.group_size * L.bits / 8);
  if constexpr (BITS == 0) {
    quantize_group(src, L.group_size, L.bits, packed, scale);
  } else {
    quantize_group_reg<T, BITS>(src, packed, scale);
  }
}

// phase 2: one workgroup per record -- CRC of the payload, header, padding.
// CHUNKED: the payload is a 16-byte multiple of at most kMaxRows rows.
template <bool CHUNKED>
__global__ __launch_bounds__(kCrcThreads) void encode_header_kernel(EncodeParams p, ChunkPlan c) {
  __shared__ ChunkLds lds;
  const Layout& L = p.lay;
  const int r = blockIdx.x;
  uint8_t* rec = p.records + static_cast<int64_t>(r) * L.record_bytes();
  uint32_t crc;
  if constexpr (CHUNKED) {
    const uint8_t* pay = rec + kHeaderBytes;
    u32x4 v[kMaxRows];
#pragma unroll
    for (int j = 0; j < kMaxRows; ++j) {
      v[j] = u32x4{0u, 0u, 0u, 0u};
      if (j < c.rows) {
        const int64_t o = chunk_offset(c, j);
        if (o >= 0) v[j] = load16(pay + o);
      }
    }
    load_chunk_tables(lds);
    __syncthreads();
    uint32_t h = 0;
#pragma unroll
    for (int j = 0; j < kMaxRows; ++j)
      if (j < c.rows) h = mul_stride(lds, h) ^ crc16_raw(lds, v[j]);
    crc = fold_chunks(lds, c, h);
  } else {
    uint32_t(*tab)[256] = lds.slice;  // the first four slicing tables
    fill_crc_tables(tab);
    __syncthreads();
    crc = block_crc32(rec + kHeaderBytes, p.plan, tab, lds.seg);
  }
  const int64_t start = static_cast<int64_t>(r) * L.block_tokens;
  const int64_t valid = p.tokens - start < L.block_tokens ? p.tokens - start : L.block_tokens;
  if (threadIdx.x < kHeaderBytes / 4) {
    uint32_t v = 0;
    switch (threadIdx.x) {
      case 0: v = kMagic0; break;
      case 1: v = kMagic1; break;
      case 2: v = 1u; break;
      case 3: v = static_cast<uint32_t>(p.layer); break;
      case 4: v = static_cast<uint32_t>(p.first_block + r); break;
      case 5: v = static_cast<uint32_t>(valid); break;
      case 6: v = static_cast<uint32_t>(L.bits); break;
      case 7: v = static_cast<uint32_t>(L.block_tokens); break;
      case 8: v = static_cast<uint32_t>(L.kv_heads); break;
      case 9: v = static_cast<uint32_t>(L.head_dim); break;
      case 10: v = static_cast<uint32_t>(L.group_size); break;
      case 11: v = p.plan.len; break;
      default: v = crc; break;
    }
    reinterpret_cast<uint32_t*>(rec)[threadIdx.x] = v;
  }
  for (int64_t i = kHeaderBytes + L.payload_bytes() + threadIdx.x; i < L.record_bytes(); i += blockDim.x) rec[i] = 0;
  if (threadIdx.x == 0) p.crcs[r] = crc;
}

// One kernel for the common layout (group size 32 in registers, the scale
// region [Ks | Vs] and the code region [Kc | Vc] each a whole number of
// 16 KiB rows of the chunked CRC form, so no virtual zeros): one workgroup of
// 1024 threads per record.  Thread t owns code chunks t, t + 1024, ... (rows
// rs .. rows - 1 of the chunked form): it quantises their groups (one INT4
// group or two INT2 groups per 16-byte chunk), stores each chunk, keeps it
// in registers and puts the scales into an LDS copy of the scale region.
// After a barrier it stores and reads back its scale chunks (rows 0 .. rs - 1)
// from LDS and folds the record's CRC-32 from registers as the gather does, so
// the payload is never read back; the header and padding follow.
struct FusedPlan {
  int rows_s, rows_c;  // rows of scale / code chunks
};

constexpr int kMaxScaleRows = 4;  // scale region <= 64 KiB of LDS
constexpr int kMaxCodeRows = 8;   // code chunks kept in registers for the CRC

template <typename T, int BITS>
__global__ __launch_bounds__(kCrcThreads) void encode_fused_kernel(EncodeParams p, ChunkPlan c, FusedPlan f) {
  __shared__ ChunkLds lds;
  __shared__ __attribute__((aligned(16))) uint16_t scales[kMaxScaleRows * kStrideBytes / 2];
  constexpr int kGroupsPerChunk = 4 / BITS;  // 32-value groups in 16 bytes of codes
  const Layout& L = p.lay;
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int G = L.head_dim / kRegGroup;
  const int64_t per_array = static_cast<int64_t>(L.block_tokens) * L.kv_heads * G;  // groups per array
  uint8_t* rec = p.records + static_cast<int64_t>(r) * L.record_bytes();
  uint8_t* pay = rec + kHeaderBytes;
  const int64_t code0 = 2 * L.scale_bytes();
  load_chunk_tables(lds);
  u32x4 code[kMaxCodeRows];
#pragma unroll
  for (int k = 0; k < kMaxCodeRows; ++k) {
    code[k] = u32x4{0u, 0u, 0u, 0u};
    if (k < f.rows_c) {
      const int64_t chunk = static_cast<int64_t>(k) * kCrcThreads + tid;  // within the code region
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < kGroupsPerChunk; ++i) {
        const int64_t q = chunk * kGroupsPerChunk + i;  // over [K groups | V groups]
        const bool is_v = q >= per_array;
        const int64_t qa = is_v ? q - per_array : q;
        const int64_t row = qa / G;  // token * kv_heads + head within the block
        const int gi = static_cast<int>(qa % G);
        const int64_t token = static_cast<int64_t>(r) * L.block_tokens + row / L.kv_heads;
        const T* base = static_cast<const T*>(is_v ? p.values : p.keys);
        const T* src =
            token < p.tokens ? base + (token * L.kv_heads + row % L.kv_heads) * L.head_dim + gi * kRegGroup : nullptr;
        const GroupWords<BITS> g = quantize_group_words<T, BITS>(src);
        constexpr int kWords = kRegGroup * BITS / 32;
#pragma unroll
        for (int k2 = 0; k2 < kWords; ++k2) w[i * kWords + k2] = g.w[k2];
        scales[q] = g.scale;
      }
      code[k] = u32x4{w[0], w[1], w[2], w[3]};
      __builtin_memcpy(__builtin_assume_aligned(pay + code0 + chunk * kChunkBytes, 4), &code[k], kChunkBytes);
    }
  }
  __syncthreads();  // every scale is in LDS (and the CRC tables)
  uint32_t h = 0;
#pragma unroll
  for (int j = 0; j < kMaxScaleRows; ++j) {
    if (j < f.rows_s) {
      const int64_t chunk = static_cast<int64_t>(j) * kCrcThreads + tid;
      const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(scales) + chunk * kChunkBytes);
      __builtin_memcpy(__builtin_assume_aligned(pay + chunk * kChunkBytes, 4), &v, kChunkBytes);
      h = mul_stride(lds, h) ^ crc16_raw(lds, v);
    }
  }
#pragma unroll
  for (int k = 0; k < kMaxCodeRows; ++k)
    if (k < f.rows_c) h = mul_stride(lds, h) ^ crc16_raw(lds, code[k]);
  const uint32_t crc = fold_chunks(lds, c, h);
  const int64_t start = static_cast<int64_t>(r) * L.block_tokens;
  const int64_t valid = p.tokens - start < L.block_tokens ? p.tokens - start : L.block_tokens;
  if (tid < kHeaderBytes / 4) {
    uint32_t v = 0;
    switch (tid) {
      case 0: v = kMagic0; break;
      case 1: v = kMagic1; break;
      case 2: v = 1u; break;
      case 3: v = static_cast<uint32_t>(p.layer); break;
      case 4: v = static_cast<uint32_t>(p.first_block + r); break;
      case 5: v = static_cast<uint32_t>(valid); break;
      case 6: v = static_cast<uint32_t>(L.bits); break;
      case 7: v = static_cast<uint32_t>(L.block_tokens); break;
      case 8: v = static_cast<uint32_t>(L.kv_heads); break;
      case 9: v = static_cast<uint32_t>(L.head_dim); break;
      case 10: v = static_cast<uint32_t>(L.group_size); break;
      case 11: v = p.plan.len; break;
      default: v = crc; break;
    }
    reinterpret_cast<uint32_t*>(rec)[tid] = v;
  }
  for (int64_t i = kHeaderBytes + L.payload_bytes() + tid; i < L.record_bytes(); i += kCrcThreads) rec[i] = 0;
  if (tid == 0) p.crcs[r] = crc;
}

// the fused form applies (register groups checked separately): scale and code
// regions whole rows of the chunked CRC form, scales within the LDS copy
bool fused_layout(const Layout& L, FusedPlan* f) {
  const int64_t sr = 2 * L.scale_bytes(), cr = 2 * L.packed_bytes();
  if (L.group_size != kRegGroup || sr % kStrideBytes || cr % kStrideBytes) return false;
  f->rows_s = static_cast<int>(sr / kStrideBytes);
  f->rows_c = static_cast<int>(cr / kStrideBytes);
  return f->rows_s >= 1 && f->rows_s <= kMaxScaleRows && f->rows_c >= 1 && f->rows_c <= kMaxCodeRows &&
         f->rows_s + f->rows_c <= kMaxRows;
}

// the chunked CRC / gather form applies: all four arrays 16-byte multiples and
// the payload at most kMaxRows rows of chunks
bool chunked_layout(const Layout& L) {
  return L.scale_bytes() % kChunkBytes == 0 && L.packed_bytes() % kChunkBytes == 0 &&
         L.payload_bytes() <= static_cast<int64_t>(kMaxRows) * kStrideBytes;
}

int check_layout(const kvssd_record_layout* l, Layout* out) {
  if (l == nullptr) return arg_error("record layout is NULL");
  if (l->bits != 2 && l->bits != 4) return arg_error("bits must be 2 or 4");
  if (l->block_tokens <= 0 || l->kv_heads <= 0 || l->head_dim <= 0)
    return arg_error("all cache dimensions must be positive");
  if (l->group_size <= 0 || l->head_dim % l->group_size) return arg_error("head_dim must be divisible by group_size");
  if (l->group_size % (8 / l->bits)) return arg_error("group_size must be positive and pack-aligned");
  *out = Layout{l->bits, l->block_tokens, l->kv_heads, l->head_dim, l->group_size};
  if (out->payload_bytes() > 0x7FFFFFFFLL) return arg_error("record payload too large");
  return 0;
}

// the register form needs group_size 32, a 16-byte aligned source and 4-byte
// aligned packed output (every group then starts aligned)
inline bool register_groups(int group_size, const void* src, const void* packed) {
  return group_size == kRegGroup && (reinterpret_cast<uintptr_t>(src) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(packed) & 3u) == 0;
}

template <typename T>
void launch_quantize_t(const void* x, int64_t groups, int group_size, int bits, uint8_t* packed, uint16_t* scales,
                       hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
  const T* src = static_cast<const T*>(x);
  if (register_groups(group_size, x, packed) && bits == 4) {
    hipLaunchKernelGGL((quantize_kernel<T, 4>), grid, dim3(256), 0, s, src, groups, group_size, bits, packed, scales);
  } else if (register_groups(group_size, x, packed) && bits == 2) {
    hipLaunchKernelGGL((quantize_kernel<T, 2>), grid, dim3(256), 0, s, src, groups, group_size, bits, packed, scales);
  } else {
    hipLaunchKernelGGL((quantize_kernel<T, 0>), grid, dim3(256), 0, s, src, groups, group_size, bits, packed, scales);
  }
}

template <typename T>
void launch_fused_t(const EncodeParams& p, const ChunkPlan& c, const FusedPlan& f, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(p.n));
  if (p.lay.bits == 4)
    hipLaunchKernelGGL((encode_fused_kernel<T, 4>), grid, dim3(kCrcThreads), 0, s, p, c, f);
  else
    hipLaunchKernelGGL((encode_fused_kernel<T, 2>), grid, dim3(kCrcThreads), 0, s, p, c, f);
}

template <typename T>
void launch_encode_t(const EncodeParams& p, hipStream_t s) {
  const int64_t groups = 2LL * p.lay.block_tokens * p.lay.kv_heads * (p.lay.head_dim / p.lay.group_size) * p.n;
  const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
  // records are 4-byte aligned (checked), so every packed group is too
  const bool reg = register_groups(p.lay.group_size, p.keys, p.records) &&
                   (reinterpret_cast<uintptr_t>(p.values) & 15u) == 0;
  if (reg && p.lay.bits == 4) {
    hipLaunchKernelGGL((encode_payload_kernel<T, 4>), grid, dim3(256), 0, s, p);
  } else if (reg && p.lay.bits == 2) {
    hipLaunchKernelGGL((encode_payload_kernel<T, 2>), grid, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((encode_payload_kernel<T, 0>), grid, dim3(256), 0, s, p);
  }
}

}  // namespace

int record_bytes_of(const kvssd_record_layout* layout, size_t* bytes) {
  Layout L{};
  if (int rc = check_layout(layout, &L)) return rc;
  if (bytes == nullptr) return arg_error("bytes output pointer is NULL");
  *bytes = static_cast<size_t>(L.record_bytes());
  return 0;
}

int launch_gather_records(const kvssd_record_layout* layout, const uint8_t* records, size_t stride, int n,
                          int verify_crc, uint8_t* packed_k, uint8_t* packed_v, uint16_t* scales_k,
                          uint16_t* scales_v, int32_t* valid, int32_t* status, hipStream_t stream) {
  Layout L{};
  if (int rc = check_layout(layout, &L)) return rc;
  if (n < 0) return arg_error("record count must be non-negative");
  if (n == 0) return 0;
  if (!records || !packed_k || !packed_v || !scales_k || !scales_v || !valid || !status)
    return arg_error("a required buffer pointer is NULL");
  if (stride < static_cast<size_t>(L.record_bytes()) || (stride % 4) || (reinterpret_cast<uintptr_t>(records) % 4))
    return arg_error("records must be 4-byte aligned and at least record_bytes apart");
  GatherParams p{};
  p.records = records;
  p.stride = static_cast<int64_t>(stride);
  p.n = n;
  p.verify = verify_crc != 0;
  p.lay = L;
  p.plan = make_crc_plan(static_cast<uint32_t>(L.payload_bytes()));
  p.pk = packed_k;
  p.pv = packed_v;
  p.sk = reinterpret_cast<uint8_t*>(scales_k);
  p.sv = reinterpret_cast<uint8_t*>(scales_v);
  p.valid = valid;
  p.status = status;
  const bool aligned16 = ((reinterpret_cast<uintptr_t>(packed_k) | reinterpret_cast<uintptr_t>(packed_v) |
                           reinterpret_cast<uintptr_t>(scales_k) | reinterpret_cast<uintptr_t>(scales_v)) & 15u) == 0;
  if (aligned16 && chunked_layout(L)) {
    const ChunkPlan c = make_chunk_plan(p.plan.len);
    hipLaunchKernelGGL(gather_chunked_kernel, dim3(static_cast<unsigned>(n)), dim3(kCrcThreads), 0, stream, p, c);
  } else {
    hipLaunchKernelGGL(gather_records_kernel, dim3(static_cast<unsigned>(n)), dim3(kCrcThreads), 0, stream, p);
  }
  return hip_status(hipGetLastError(), "gather_records launch");
}

int launch_quantize(const void* x, int dtype, int64_t rows, int head_dim, int bits, int group_size, uint8_t* packed,
                    uint16_t* scales, hipStream_t stream) {
  if (bits != 2 && bits != 4) return arg_error("bits must be 2 or 4");
  if (group_size <= 0 || group_size % (8 / bits)) return arg_error("group_size must be positive and pack-aligned");
  if (head_dim <= 0 || head_dim % group_size) return arg_error("last dimension must be divisible by group_size");
  if (rows < 0) return arg_error("row count must be non-negative");
  if (rows == 0) return 0;
  if (!x || !packed || !scales) return arg_error("a required buffer pointer is NULL");
  const int64_t groups = rows * (head_dim / group_size);
  switch (dtype) {
    case KVSSD_DTYPE_F16:
      launch_quantize_t<_Float16>(x, groups, group_size, bits, packed, scales, stream);
      break;
    case KVSSD_DTYPE_BF16:
      launch_quantize_t<uint16_t>(x, groups, group_size, bits, packed, scales, stream);
      break;
    case KVSSD_DTYPE_F32:
      launch_quantize_t<float>(x, groups, group_size, bits, packed, scales, stream);
      break;
    case KVSSD_DTYPE_F64:
      launch_quantize_t<double>(x, groups, group_size, bits, packed, scales, stream);
      break;
    default:
      return arg_error("quantization input must be floating point");
  }
  return hip_status(hipGetLastError(), "quantize launch");
}

int launch_encode_records(const kvssd_record_layout* layout, int dtype, const void* keys, const void* values,
                          int64_t tokens, int layer, int first_block, uint8_t* records, uint32_t* crcs,
                          hipStream_t stream) {
  Layout L{};
  if (int rc = check_layout(layout, &L)) return rc;
  if (tokens < 0) return arg_error("token count must be non-negative");
  if (tokens == 0) return 0;
  if (!keys || !values || !records || !crcs) return arg_error("a required buffer pointer is NULL");
  if (reinterpret_cast<uintptr_t>(records) % 4) return arg_error("records must be 4-byte aligned");
  EncodeParams p{};
  p.keys = keys;
  p.values = values;
  p.tokens = tokens;
  p.n = static_cast<int>((tokens + L.block_tokens - 1) / L.block_tokens);
  p.layer = layer;
  p.first_block = first_block;
  p.lay = L;
  p.plan = make_crc_plan(static_cast<uint32_t>(L.payload_bytes()));
  p.records = records;
  p.crcs = crcs;
  const uint32_t len = p.plan.len;
  const ChunkPlan c = make_chunk_plan(len);
  FusedPlan f{};
  // (fp64 input keeps the two-kernel form: its fused INT2 instance would spill)
  if (fused_layout(L, &f) && register_groups(L.group_size, keys, records) &&
      (reinterpret_cast<uintptr_t>(values) & 15u) == 0 &&
      (dtype == KVSSD_DTYPE_F16 || dtype == KVSSD_DTYPE_BF16 || dtype == KVSSD_DTYPE_F32)) {
    if (dtype == KVSSD_DTYPE_F16) launch_fused_t<_Float16>(p, c, f, stream);
    else if (dtype == KVSSD_DTYPE_BF16) launch_fused_t<uint16_t>(p, c, f, stream);
    else launch_fused_t<float>(p, c, f, stream);
    return hip_status(hipGetLastError(), "encode_records launch");
  }
  switch (dtype) {
    case KVSSD_DTYPE_F16:
      launch_encode_t<_Float16>(p, stream);
      break;
    case KVSSD_DTYPE_BF16:
      launch_encode_t<uint16_t>(p, stream);
      break;
    case KVSSD_DTYPE_F32:
      launch_encode_t<float>(p, stream);
      break;
    case KVSSD_DTYPE_F64:
      launch_encode_t<double>(p, stream);
      break;
    default:
      return arg_error("quantization input must be floating point");
  }
  if (int rc = hip_status(hipGetLastError(), "encode_records launch")) return rc;
  if (len % kChunkBytes == 0 && c.rows <= kMaxRows) {
    hipLaunchKernelGGL(encode_header_kernel<true>, dim3(static_cast<unsigned>(p.n)), dim3(kCrcThreads), 0, stream, p, c);
  } else {
    hipLaunchKernelGGL(encode_header_kernel<false>, dim3(static_cast<unsigned>(p.n)), dim3(kCrcThreads), 0, stream, p, c);
  }
  return hip_status(hipGetLastError(), "encode_records launch");
}

}  // namespace kvssd
