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

}  // namespace

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
