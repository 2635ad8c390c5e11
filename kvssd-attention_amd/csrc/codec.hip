// Bit-exact codec twins used to check the kernels' in-register unpack.
//
// unpack_codes runs the same magic-number unpack the matrix-core kernel feeds
// its MFMA operands with (common.hpp: unpack_int4_f16 / unpack_int2_f16), then
// reads each fp16 lane back through a hardware fp16 -> fp32 conversion:
//   code = F * (value - 1)   (value = 1 + code / F, F = 64 for INT4, 4 for INT2)
// so any mistake in which code lands in which fp16 lane, or in the exponent
// and mantissa placement, changes the output.  Twin of unpack_codes
// (src/kvssd/quant.py:40-46).
//
// dequantize: (code - mid) * fp16 scale in fp32, the operation of
// dequantize_tensor (src/kvssd/quant.py:68-73) and of
// csrc/fused_decode.cu:53-56; exact in fp32.
#include "decode.hpp"

namespace kvssd {
namespace {

__device__ __forceinline__ uint8_t code_from_f16(uint32_t word, int hi, float codes_per_unit) {
  const uint16_t bits = static_cast<uint16_t>(hi ? (word >> 16) : (word & 0xFFFFu));
  const float value = half_bits_to_float(bits);
  return static_cast<uint8_t>(__float2int_rn((value - 1.0f) * codes_per_unit));
}

// One thread per 32-bit word of packed bytes (8 INT4 or 16 INT2 codes);
// the tail (n_bytes % 4) is handled by the last thread with byte loads.
__global__ void unpack_codes_kernel(const uint8_t* __restrict__ packed, int bits, int64_t n_bytes,
                                    uint8_t* __restrict__ codes) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t first = w * 4;
  if (first >= n_bytes) return;
  uint32_t x = 0;
  const int avail = static_cast<int>(n_bytes - first < 4 ? n_bytes - first : 4);
  for (int i = 0; i < avail; ++i) x |= static_cast<uint32_t>(packed[first + i]) << (8 * i);
  if (bits == 4) {
    uint32_t f[4];
    unpack_int4_f16(x, f);
    uint8_t c[8];
    // f[j] = (n_j, n_{j+4})
    for (int j = 0; j < 4; ++j) {
      c[j] = code_from_f16(f[j], 0, kUnpackScale<4>);
      c[j + 4] = code_from_f16(f[j], 1, kUnpackScale<4>);
    }
    for (int i = 0; i < 2 * avail; ++i) codes[first * 2 + i] = c[i];
  } else {
    uint32_t f[8];
    unpack_int2_f16(x, f);
    uint8_t c[16];
    // f[j] = (c_j, c_{j+8})
    for (int j = 0; j < 8; ++j) {
      c[j] = code_from_f16(f[j], 0, kUnpackScale<2>);
      c[j + 8] = code_from_f16(f[j], 1, kUnpackScale<2>);
    }
    for (int i = 0; i < 4 * avail; ++i) codes[first * 4 + i] = c[i];
  }
}

__global__ void dequantize_kernel(const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales,
                                  int64_t rows, int head_dim, int bits, int group_size, float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * head_dim) return;
  const int64_t row = i / head_dim;
  const int dd = static_cast<int>(i % head_dim);
  const int per = 8 / bits;
  const int packed_dim = head_dim * bits / 8;
  const int code = (packed[row * packed_dim + dd / per] >> ((dd % per) * bits)) & ((1 << bits) - 1);
  const int mid = 1 << (bits - 1);
  out[i] = static_cast<float>(code - mid) * half_bits_to_float(scales[row * (head_dim / group_size) + dd / group_size]);
}

// Streaming read of n16 16-byte chunks: the plain HBM read rate a decode's
// packed-KV traffic is measured against.  A workgroup reads contiguous
// 32 KB pieces (eight 16-byte non-temporal loads in flight per thread, the
// hint the decode kernels' code copies carry), the grid striding over the
// buffer; the chunks fold by XOR and every wave leaves one dword in `sink`,
// so no load can be elided.  (Measured on MI355X over 1 GiB: this shape
// 7.0 TB/s; loads a whole grid apart 5.7 TB/s; without the hint 6.2 TB/s.)
constexpr int kProbeThreads = 256;
constexpr int kProbeBlocks = 2048;
constexpr int kProbeUnroll = 8;
typedef uint32_t probe_u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const probe_u32x4* __restrict__ p, int64_t n16,
                                                                   uint32_t* __restrict__ sink) {
  constexpr int64_t kPiece = kProbeThreads * kProbeUnroll;  // 16-byte chunks per workgroup pass
  probe_u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kPiece; base < n16;
       base += static_cast<int64_t>(gridDim.x) * kPiece) {
    if (base + kPiece <= n16) {
      probe_u32x4 v[kProbeUnroll];
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(p + base + u * kProbeThreads + threadIdx.x);
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
    } else {
      for (int64_t i = base + threadIdx.x; i < n16; i += kProbeThreads) acc ^= p[i];
    }
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  for (int m = 32; m > 0; m >>= 1) x ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), m, kWave));
  if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (kProbeThreads / kWave) + threadIdx.x / kWave] = x;
}

}  // namespace

size_t read_probe_sink_words() { return static_cast<size_t>(kProbeBlocks) * (kProbeThreads / kWave); }

int launch_read_probe(const void* data, size_t bytes, uint32_t* sink, hipStream_t stream) {
  if (bytes == 0) return 0;
  hipLaunchKernelGGL(read_probe_kernel, dim3(kProbeBlocks), dim3(kProbeThreads), 0, stream,
                     static_cast<const probe_u32x4*>(data), static_cast<int64_t>(bytes / 16), sink);
  return hip_status(hipGetLastError(), "read_probe launch");
}

int launch_unpack_codes(const uint8_t* packed, int bits, int64_t n_bytes, uint8_t* codes, hipStream_t stream) {
  if (n_bytes <= 0) return 0;
  const int64_t words = (n_bytes + 3) / 4;
  const int threads = 256;
  const int64_t blocks = (words + threads - 1) / threads;
  hipLaunchKernelGGL(unpack_codes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, stream, packed, bits,
                     n_bytes, codes);
  return hip_status(hipGetLastError(), "unpack_codes launch");
}

int launch_dequantize(const uint8_t* packed, const uint16_t* scales, int64_t rows, int head_dim, int bits,
                      int group_size, float* out, hipStream_t stream) {
  const int64_t n = rows * head_dim;
  if (n <= 0) return 0;
  const int threads = 256;
  const int64_t blocks = (n + threads - 1) / threads;
  hipLaunchKernelGGL(dequantize_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, stream, packed, scales,
                     rows, head_dim, bits, group_size, out);
  return hip_status(hipGetLastError(), "dequantize launch");
}

}  // namespace kvssd
