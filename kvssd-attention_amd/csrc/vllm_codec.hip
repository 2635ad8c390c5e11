// vLLM block codec on the GPU (src/kvssd/integrations/vllm_codec.py:42-102).
//
// A record is a 32-byte header "<8sBBBBIIQI" (magic "KVVLLM02", version 1,
// bits, dtype code, reserved 0, group_size, elements, payload bytes, CRC-32 of
// the payload), the payload -- fp16 scales [elements / group_size] then the
// packed codes [elements * bits / 8] of the block's values taken as one flat
// vector -- and zero padding to a 4096 multiple.
//
// * encode: the block is quantised straight into the payload (the same
//   kernels as quantize_tensor's twin), then the payload CRC, the header and
//   the padding;
// * decode: the caller has checked the header on the host (it holds the
//   reference's ValueErrors); the GPU verifies the payload CRC and
//   dequantises the codes into the destination, (code - mid) * scale in fp32
//   rounded once to the destination dtype, as dequantize_tensor(..., dtype).
//
// The CRC runs over many workgroups: workgroup r takes row r of 1024 16-byte
// chunks (the payload virtually left-padded with zeros to whole rows), folds
// it to one raw register value, and one workgroup folds the row values.
#include "crc32.hpp"
#include "decode.hpp"

namespace kvssd {
namespace {

constexpr int kVHeader = 32;
constexpr int kVAlign = 4096;
constexpr int kMaxVRows = kCrcThreads;  // payload <= 1024 rows of 16 KiB
constexpr uint32_t kVMagic0 = 0x4C56564Bu;  // "KVVL", little-endian
constexpr uint32_t kVMagic1 = 0x32304D4Cu;  // "LM02"

struct VPlan {
  uint32_t len;                   // payload bytes
  int rows;                       // rows of 1024 16-byte chunks
  int64_t pad;                    // leading virtual zero bytes
  bool wide;                      // len % 16 == 0 and the payload 4-byte aligned: 16-byte loads
  uint32_t x_len;                 // x^(8 len)
};

struct VShape {
  int64_t elements;
  int bits, group_size;
  int64_t scale_bytes;  // 2 * elements / group_size
};

VPlan make_vplan(uint32_t len, const uint8_t* payload) {
  VPlan v{};
  v.len = len;
  v.rows = static_cast<int>((len + kStrideBytes - 1) / kStrideBytes);
  if (v.rows == 0) v.rows = 1;
  v.pad = static_cast<int64_t>(v.rows) * kStrideBytes - len;
  v.wide = (len % kChunkBytes) == 0 && (reinterpret_cast<uintptr_t>(payload) & 3u) == 0;
  v.x_len = x_pow_bytes(len);
  return v;
}

__device__ __forceinline__ float half_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// The codes of packed bytes [q0, q0 + 16) (q0 >= 0: every byte is a packed
// byte) dequantised into dst: (code - mid) * scale in fp32, one rounding.
// The group index is tracked along the chunk (one division per chunk) and the
// chunk's values go out in one wide store when the destination allows it.
template <typename T, int BITS>
__device__ __forceinline__ void dequant_chunk(const uint8_t* payload, const VShape& sh, u32x4 v, int64_t q0, T* dst) {
  constexpr int per = 8 / BITS;
  constexpr int n = kChunkBytes * per;
  constexpr int mid = 1 << (BITS - 1);
  constexpr uint32_t mask = (1u << BITS) - 1u;
  const uint16_t* scales = reinterpret_cast<const uint16_t*>(payload);
  const uint32_t e0 = static_cast<uint32_t>(q0 * per);  // elements < 2^32
  const uint32_t g = static_cast<uint32_t>(sh.group_size);
  uint32_t sidx = e0 / g, rr = e0 - sidx * g;
  float sc = half_to_f32(scales[sidx]);
  T out[n];
#pragma unroll
  for (int i = 0; i < n; ++i) {
    const uint32_t byte = (v[i / per / 4] >> (8 * ((i / per) & 3))) & 0xFFu;
    const int code = static_cast<int>((byte >> ((i % per) * BITS)) & mask);
    out[i] = store_cast<T>(static_cast<float>(code - mid) * sc);
    if (++rr == g && i + 1 < n) {
      rr = 0;
      sc = half_to_f32(scales[++sidx]);
    }
  }
  T* d = dst + e0;
  if ((reinterpret_cast<uintptr_t>(d) & 15u) == 0) {
    __builtin_memcpy(__builtin_assume_aligned(d, 16), out, sizeof(out));
  } else {
#pragma unroll
    for (int i = 0; i < n; ++i) d[i] = out[i];
  }
}

// Row r of the payload: this thread's 16-byte chunk, its raw CRC folded over
// the row into parts[r].  BITS != 0: the codes in the chunk are also
// dequantised into DST (elements indexed as the flat block).
template <typename T, int BITS>
__global__ __launch_bounds__(kCrcThreads) void vllm_rows_kernel(const uint8_t* __restrict__ payload, VPlan pl, VShape sh,
                                                                T* __restrict__ dst, uint32_t* __restrict__ parts) {
  __shared__ ChunkLds lds;
  load_chunk_tables(lds);
  const int64_t o = (static_cast<int64_t>(blockIdx.x) * kCrcThreads + threadIdx.x) * kChunkBytes - pl.pad;
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (pl.wide) {
    if (o >= 0) v = load16(payload + o);
  } else {
    // the chunk ends inside the payload (o + 15 < len); bytes before 0 are virtual zeros
#pragma unroll
    for (int k = 0; k < kChunkBytes; ++k) {
      const uint32_t b = (o + k >= 0) ? payload[o + k] : 0u;
      v[k >> 2] |= b << (8 * (k & 3));
    }
  }
  __syncthreads();  // tables in LDS
  const uint32_t h = crc16_raw(lds, v);
  if constexpr (BITS != 0) {
    const int64_t q0 = o - sh.scale_bytes;  // first byte of the chunk in the packed region
    if (q0 >= 0) {
      dequant_chunk<T, BITS>(payload, sh, v, q0, dst);
    } else if (q0 + kChunkBytes > 0) {
      // the chunk holding the end of the scales (or of the virtual zeros)
      constexpr int per = 8 / BITS;
      for (int k = static_cast<int>(-q0); k < kChunkBytes; ++k) {
        const uint32_t byte = (v[k >> 2] >> (8 * (k & 3))) & 0xFFu;
        for (int j = 0; j < per; ++j) {
          const int64_t e = (q0 + k) * per + j;
          const uint16_t sc = reinterpret_cast<const uint16_t*>(payload)[e / sh.group_size];
          const int code = static_cast<int>((byte >> (j * BITS)) & ((1u << BITS) - 1u));
          dst[e] = store_cast<T>(static_cast<float>(code - (1 << (BITS - 1))) * half_to_f32(sc));
        }
      }
    }
  }
  const uint32_t raw = fold_pos(lds, kPosTables.chunk, h);
  if (threadIdx.x == 0) parts[blockIdx.x] = raw;
}

// One workgroup: the payload CRC from the row values.  ENCODE: write the
// header (fields in hdr2/hdr3/hdr4: version|bits|dtype|0, group_size,
// elements) and the zero padding of `record`, and the CRC to *crc_out.
// Otherwise: *status = 0 if the CRC equals `expected`, else 3.
template <bool ENCODE>
__global__ __launch_bounds__(kCrcThreads) void vllm_combine_kernel(const uint32_t* __restrict__ parts, VPlan pl,
                                                                   uint8_t* __restrict__ record, uint32_t hdr2,
                                                                   uint32_t hdr3, uint32_t hdr4, int64_t record_bytes,
                                                                   uint32_t expected, int32_t* __restrict__ status,
                                                                   uint32_t* __restrict__ crc_out) {
  __shared__ ChunkLds lds;
  const int t = threadIdx.x;
  const int lead = kCrcThreads - pl.rows;  // leading zero rows leave the raw register unchanged
  const uint32_t h = t >= lead ? parts[t - lead] : 0u;
  const uint32_t crc = crc_from_raw(pl.x_len, fold_pos(lds, kPosTables.row, h));
  if constexpr (ENCODE) {
    if (t < kVHeader / 4) {
      uint32_t w = 0;
      switch (t) {
        case 0: w = kVMagic0; break;
        case 1: w = kVMagic1; break;
        case 2: w = hdr2; break;
        case 3: w = hdr3; break;
        case 4: w = hdr4; break;
        case 5: w = pl.len; break;  // payload bytes, low word
        case 6: w = 0u; break;      // high word
        default: w = crc; break;
      }
      reinterpret_cast<uint32_t*>(record)[t] = w;
    }
    for (int64_t i = kVHeader + pl.len + t; i < record_bytes; i += kCrcThreads) record[i] = 0;
    if (t == 0) crc_out[0] = crc;
  } else {
    if (t == 0) {
      status[0] = crc == expected ? 0 : 3;
      if (crc_out != nullptr) crc_out[0] = crc;
    }
  }
}

int check_vshape(int64_t elements, int bits, int group_size, VShape* sh, uint32_t* len) {
  if (bits != 2 && bits != 4) return arg_error("bits must be 2 or 4");
  if (group_size <= 0 || group_size % (8 / bits)) return arg_error("group_size must be positive and pack-aligned");
  if (elements <= 0) return arg_error("a vLLM block must hold at least one value");
  if (elements % group_size)
    return arg_error("vLLM block has " + std::to_string(elements) + " values, not divisible by group_size=" +
                     std::to_string(group_size));
  if (elements > 0xFFFFFFFFLL) return arg_error("a vLLM block holds at most 2^32 - 1 values");
  const int64_t payload = elements / group_size * 2 + elements * bits / 8;
  if (payload > static_cast<int64_t>(kMaxVRows) * kStrideBytes) return arg_error("vLLM block payload above 16 MiB");
  *sh = VShape{elements, bits, group_size, elements / group_size * 2};
  *len = static_cast<uint32_t>(payload);
  return 0;
}

int64_t vrecord_bytes(uint32_t len) { return (kVHeader + static_cast<int64_t>(len) + kVAlign - 1) / kVAlign * kVAlign; }

// dtype code of the vLLM header (vllm_codec.py:19): float16 1, bfloat16 2, float32 3
int vllm_dtype_code(int dtype) {
  switch (dtype) {
    case KVSSD_DTYPE_F16: return 1;
    case KVSSD_DTYPE_BF16: return 2;
    case KVSSD_DTYPE_F32: return 3;
    default: return 0;
  }
}

template <typename T, int BITS>
void launch_rows(const uint8_t* payload, const VPlan& pl, const VShape& sh, void* dst, uint32_t* parts, hipStream_t s) {
  hipLaunchKernelGGL((vllm_rows_kernel<T, BITS>), dim3(static_cast<unsigned>(pl.rows)), dim3(kCrcThreads), 0, s, payload,
                     pl, sh, static_cast<T*>(dst), parts);
}

template <typename T>
void launch_rows_bits(const uint8_t* payload, const VPlan& pl, const VShape& sh, void* dst, uint32_t* parts,
                      hipStream_t s) {
  if (sh.bits == 4) launch_rows<T, 4>(payload, pl, sh, dst, parts, s);
  else launch_rows<T, 2>(payload, pl, sh, dst, parts, s);
}

}  // namespace

int vllm_sizes(int64_t elements, int bits, int group_size, size_t* record_bytes, size_t* scratch_bytes) {
  VShape sh{};
  uint32_t len = 0;
  if (int rc = check_vshape(elements, bits, group_size, &sh, &len)) return rc;
  if (record_bytes) *record_bytes = static_cast<size_t>(vrecord_bytes(len));
  if (scratch_bytes) *scratch_bytes = static_cast<size_t>((len + kStrideBytes - 1) / kStrideBytes) * 4 + 4;
  return 0;
}

int launch_vllm_encode(const void* values, int dtype, int64_t elements, int bits, int group_size, uint8_t* record,
                       uint32_t* crc, void* scratch, size_t scratch_bytes, hipStream_t stream) {
  VShape sh{};
  uint32_t len = 0;
  if (int rc = check_vshape(elements, bits, group_size, &sh, &len)) return rc;
  const int code = vllm_dtype_code(dtype);
  if (code == 0) return arg_error("vLLM blocks hold float16, bfloat16 or float32 values");
  if (!values || !record || !crc || !scratch) return arg_error("a required buffer pointer is NULL");
  if (reinterpret_cast<uintptr_t>(record) % 4) return arg_error("record must be 4-byte aligned");
  size_t need = 0;
  vllm_sizes(elements, bits, group_size, nullptr, &need);
  if (scratch_bytes < need) return arg_error("scratch buffer too small for this vLLM block");
  uint8_t* payload = record + kVHeader;
  // one group per row of group_size values: the flat block's groups
  if (int rc = launch_quantize(values, dtype, elements / group_size, group_size, bits, group_size,
                               payload + sh.scale_bytes, reinterpret_cast<uint16_t*>(payload), stream))
    return rc;
  const VPlan pl = make_vplan(len, payload);
  uint32_t* parts = static_cast<uint32_t*>(scratch);
  launch_rows<float, 0>(payload, pl, sh, nullptr, parts, stream);
  if (int rc = hip_status(hipGetLastError(), "vllm encode rows launch")) return rc;
  const uint32_t hdr2 = 1u | (static_cast<uint32_t>(bits) << 8) | (static_cast<uint32_t>(code) << 16);
  hipLaunchKernelGGL(vllm_combine_kernel<true>, dim3(1), dim3(kCrcThreads), 0, stream, parts, pl, record, hdr2,
                     static_cast<uint32_t>(group_size), static_cast<uint32_t>(elements), vrecord_bytes(len), 0u,
                     static_cast<int32_t*>(nullptr), crc);
  return hip_status(hipGetLastError(), "vllm encode combine launch");
}

int launch_vllm_decode(const uint8_t* payload, int64_t elements, int bits, int group_size, uint32_t expected_crc,
                       int dtype, void* destination, int32_t* status, void* scratch, size_t scratch_bytes,
                       hipStream_t stream) {
  VShape sh{};
  uint32_t len = 0;
  if (int rc = check_vshape(elements, bits, group_size, &sh, &len)) return rc;
  if (vllm_dtype_code(dtype) == 0) return arg_error("vLLM blocks hold float16, bfloat16 or float32 values");
  if (!payload || !destination || !status || !scratch) return arg_error("a required buffer pointer is NULL");
  size_t need = 0;
  vllm_sizes(elements, bits, group_size, nullptr, &need);
  if (scratch_bytes < need) return arg_error("scratch buffer too small for this vLLM block");
  const VPlan pl = make_vplan(len, payload);
  uint32_t* parts = static_cast<uint32_t*>(scratch);
  switch (dtype) {
    case KVSSD_DTYPE_F16:
      launch_rows_bits<_Float16>(payload, pl, sh, destination, parts, stream);
      break;
    case KVSSD_DTYPE_BF16:
      launch_rows_bits<uint16_t>(payload, pl, sh, destination, parts, stream);
      break;
    default:
      launch_rows_bits<float>(payload, pl, sh, destination, parts, stream);
      break;
  }
  if (int rc = hip_status(hipGetLastError(), "vllm decode rows launch")) return rc;
  hipLaunchKernelGGL(vllm_combine_kernel<false>, dim3(1), dim3(kCrcThreads), 0, stream, parts, pl,
                     static_cast<uint8_t*>(nullptr), 0u, 0u, 0u, int64_t{0}, expected_crc, status,
                     static_cast<uint32_t*>(nullptr));
  return hip_status(hipGetLastError(), "vllm decode combine launch");
}

}  // namespace kvssd
