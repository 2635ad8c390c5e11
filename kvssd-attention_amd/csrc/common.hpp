// Shared host/device helpers of libkvssd_hip.so (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/kvssd_hip.h"

namespace kvssd {

// ---------------------------------------------------------------- errors ---

// Argument errors are negative, runtime errors are the positive hipError_t.
constexpr int kArgError = -1;

void set_error(const std::string& msg);
int arg_error(const std::string& msg);
int hip_status(hipError_t err, const char* what);

// ------------------------------------------------------------- constants ---

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kWave = 64;

// Workspace of a split decode: per (split, query head) an unnormalised fp32
// output row O[D] plus (m, l), m the running max in log2 units and l the sum of
// 2^(s - m) over the split's tokens.
struct SplitPartials {
  float* o;   // [splits][query_heads][head_dim]
  float* ml;  // [splits][query_heads][2]
};

inline size_t split_partial_bytes(int splits, int query_heads, int head_dim) {
  size_t rows = static_cast<size_t>(splits) * query_heads;
  size_t o = rows * head_dim * sizeof(float);
  o = (o + 255) & ~static_cast<size_t>(255);
  return o + rows * 2 * sizeof(float);
}

inline SplitPartials carve_partials(void* ws, int splits, int query_heads, int head_dim) {
  size_t rows = static_cast<size_t>(splits) * query_heads;
  size_t o = rows * head_dim * sizeof(float);
  o = (o + 255) & ~static_cast<size_t>(255);
  auto* base = static_cast<char*>(ws);
  return SplitPartials{reinterpret_cast<float*>(base), reinterpret_cast<float*>(base + o)};
}

// ------------------------------------------------------------ device side ---

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

template <typename QT>
__device__ __forceinline__ float load_query(const void* q, int index);

template <>
__device__ __forceinline__ float load_query<_Float16>(const void* q, int index) {
  return static_cast<float>(static_cast<const _Float16*>(q)[index]);
}
template <>
__device__ __forceinline__ float load_query<uint16_t>(const void* q, int index) {  // bfloat16 bits
  uint32_t bits = static_cast<uint32_t>(static_cast<const uint16_t*>(q)[index]) << 16;
  return __builtin_bit_cast(float, bits);
}
template <>
__device__ __forceinline__ float load_query<float>(const void* q, int index) {
  return static_cast<const float*>(q)[index];
}
template <>
__device__ __forceinline__ float load_query<double>(const void* q, int index) {
  return static_cast<float>(static_cast<const double*>(q)[index]);
}

// fp32 -> storage of a destination dtype, rounded to nearest even (the
// rounding of torch's Tensor.to for these types; bf16 NaN -> 0x7FC0)
template <typename T>
__device__ __forceinline__ T store_cast(float x);
template <>
__device__ __forceinline__ _Float16 store_cast<_Float16>(float x) {
  return static_cast<_Float16>(x);
}
template <>
__device__ __forceinline__ float store_cast<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ double store_cast<double>(float x) {
  return static_cast<double>(x);
}
template <>
__device__ __forceinline__ uint16_t store_cast<uint16_t>(float x) {  // bfloat16 bits
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;  // NaN
  return static_cast<uint16_t>((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// Rows of a block that take part in attention for its count v: the rows
// Python's slice keys[block, :v] keeps (src/kvssd/backends/reference.py:38-40),
// i.e. min(v, BT) for v >= 0 and max(BT + v, 0) for v < 0.
__device__ __forceinline__ int clamp_valid(int v, int block_tokens) {
  const int n = v < 0 ? block_tokens + v : v;
  return n < 0 ? 0 : (n > block_tokens ? block_tokens : n);
}

// --- in-register unpack of packed codes into fp16 pairs (magic numbers) ---
//
// A code c sits in the mantissa of an fp16 whose exponent field is that of
// 1.0 (0x3C00):
//   INT4: bits 4..7  -> value 1 + c/64, so c - 8 = 64 * (value - 1.125)
//   INT2: bits 8..9  -> value 1 + c/4,  so c - 2 =  4 * (value - 1.5)
// i.e. (c - mid) = F * (value - (1 + mid/F)) with F = kUnpackScale<bits>.
// Each output word holds two fp16 lanes (lo, hi): one AND-OR per word plus at
// most one shift (INT4: 3 shifts per 4 words' worth of 8 nibbles).
//
// INT4, x holds nibbles n0..n7 (n_i = bits 4i..4i+3, i.e. dims d0..d7 of a
// packed row, low bits first):
//   w0 = (n0, n4), w1 = (n1, n5), w2 = (n2, n6), w3 = (n3, n7).
// INT2, x holds codes c0..c15 (bits 2i..2i+1):
//   w_j = (c_j, c_{j+8}) for j = 0..7.
constexpr uint32_t kF16One2 = 0x3C003C00u;
constexpr uint32_t kMaskInt4 = 0x00F000F0u;
constexpr uint32_t kMaskInt2 = 0x03000300u;
template <int BITS>
constexpr float kUnpackScale = BITS == 4 ? 64.0f : 4.0f;     // F
template <int BITS>
constexpr float kUnpackOffset = BITS == 4 ? 1.125f : 1.5f;  // 1 + mid/F

// (x & m) | c.  Plain C on purpose: the backend emits v_and_b32 + v_or_b32
// for it, and an inline-asm v_and_or_b32 is invisible to the compiler's hazard
// recognizer, so a VALU result feeding an MFMA operand could be read without
// the wait states the hardware needs (that produced wrong MFMA results here).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }

__device__ __forceinline__ void unpack_int4_f16(uint32_t x, uint32_t w[4]) {
  const uint32_t m = kMaskInt4;
  w[0] = and_or(x << 4, m, kF16One2);
  w[1] = and_or(x, m, kF16One2);
  w[2] = and_or(x >> 4, m, kF16One2);
  w[3] = and_or(x >> 8, m, kF16One2);
}

__device__ __forceinline__ void unpack_int2_f16(uint32_t x, uint32_t w[8]) {
  const uint32_t m = kMaskInt2;
  w[0] = and_or(x << 8, m, kF16One2);
  w[1] = and_or(x << 6, m, kF16One2);
  w[2] = and_or(x << 4, m, kF16One2);
  w[3] = and_or(x << 2, m, kF16One2);
  w[4] = and_or(x, m, kF16One2);
  w[5] = and_or(x >> 2, m, kF16One2);
  w[6] = and_or(x >> 4, m, kF16One2);
  w[7] = and_or(x >> 6, m, kF16One2);
}

// --- DPP row (16-lane) reductions: v_max/v_add with row_ror operands ---
template <int kRor>
__device__ __forceinline__ float row_ror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + kRor, 0xF, 0xF,
                                                               false));
}
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<1>(v));
  return v;
}
__device__ __forceinline__ float row_sum16(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

// Max / sum over the 64 lanes of a wave (every lane active), in every lane:
// DPP rotations inside each 16-lane row, then the four row results through
// v_readlane -- VALU only, where a shuffle (ds_bpermute) pays an LDS round
// trip per step.
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row_max16(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// --- V-scale exponent of a stage (the matrix-core kernels' fp16 W) ---
//
// The matrix-core kernels form W = p * scale_v in fp16 for the PV product.
// p = 2^(s - m) <= 1, but scale_v spans fp16's whole range: W can overflow
// (up to 65504 / 7 for INT4 scales, times a slot factor of up to 16) or fall
// into fp16's subnormals (scale_v below ~6e-5: W loses its precision).  So
// each stage (sub-block) takes e = E - 10, E the exponent of its largest
// |scale_v| (|scale_v| < 2^(E+1)), and forms W = 2^(s - (m + e)) * scale_v:
// every W is at most 2^11 (2^15 with the slot factor), and a token whose
// weight 2^s * scale_v lies within 2^24 of the stage's largest possible one
// stays a normal fp16 number.  The 2^-e rides on the softmax reference point:
// the running (m, l, O) of a wave are all relative to m + e, so O / l is
// unchanged, a stage whose m + e is larger rescales the state like a larger
// max does, and lse = ln 2 (m + e + log2 l) as before.

// Largest |x| over the four fp16 values of w, as fp16 bits (sign cleared,
// so the integer order is the magnitude order; NaN and inf sort last).
__device__ __forceinline__ uint32_t abs_max_bits(uint32_t w0, uint32_t w1) {
  typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
  const u16x2 m = __builtin_elementwise_max(__builtin_bit_cast(u16x2, w0 & 0x7FFF7FFFu),
                                            __builtin_bit_cast(u16x2, w1 & 0x7FFF7FFFu));
  const uint32_t lo = m[0], hi = m[1];
  return lo > hi ? lo : hi;
}

// e = E - 10 for the largest of the wave's fp16 magnitude bits x (every lane
// active; wave-uniform): DPP row rotations, then the four rows through
// v_readlane.  s_nop 1 before each DPP read covers the VALU-write -> DPP-read
// hazard (two wait states); nothing here involves the matrix core.  A zero or
// subnormal maximum counts as 2^-14 (e = -24), inf and NaN as 2^16 (e = 6).
__device__ __forceinline__ int wave_scale_exp(uint32_t x) {
  uint32_t r;
  asm("s_nop 1\n\t"
      "v_max_u32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_ror:2 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_u32_dpp %0, %0, %0 row_ror:1 row_mask:0xf bank_mask:0xf"
      : "=&v"(r)
      : "v"(x));
  const int ri = static_cast<int>(r);
  const int a = max(max(__builtin_amdgcn_readlane(ri, 0), __builtin_amdgcn_readlane(ri, 16)),
                    max(__builtin_amdgcn_readlane(ri, 32), __builtin_amdgcn_readlane(ri, 48)));
  return max(a >> 10, 1) - 25;
}

// v from the lane of this lane's quad given by the DPP quad_perm control
template <int kQuadPerm>
__device__ __forceinline__ float quad_lane(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kQuadPerm, 0xF, 0xF,
                                                               false));
}

}  // namespace kvssd
