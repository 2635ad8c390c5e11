// Internal launch interface between the C ABI (abi.hip) and the kernels.
#pragma once

#include "common.hpp"

namespace kvssd {

struct DecodeArgs {
  kvssd_decode_desc desc;
  const void* query;
  const uint8_t* packed_k;
  const uint8_t* packed_v;
  const uint16_t* scales_k;
  const uint16_t* scales_v;
  const int32_t* valid;
  const int32_t* table;  // nullptr: identity over num_blocks
  int units;             // blocks attended (num_selected or num_blocks)
  hipStream_t stream;
};

// ---- kernel arguments of the matrix-core kernels.  Their first nine
// arguments (query, pk, pv, sk, sv and the four dwords below: 14 dwords, what
// the first loads need) arrive preloaded in SGPRs at wave launch (the library
// is built with -amdgpu-kernarg-preload-count), so no load waits for a
// kernel-argument fetch; these 12 come from the kernel-argument segment in
// two scalar loads issued at entry.  Every dword is used (`splits` fills the
// second load in a kernel that has no use for it): the compiler reuses the
// register of a dead dword at once, and writing a pending load's destination
// waits for the load.
struct DecodeTail {
  const int32_t* valid;
  const int32_t* table;
  float* part_o;
  float* part_ml;
  int query_heads, num_blocks;
  float scale_log2;  // sm_scale * log2(e)
  int splits;
};
// heads argument: kv_heads in bits 0-15, query heads per kv head in 16-23,
// bit 24 set when there is a block table, bit 25 when each of a kv head's two
// query quads gets a workgroup of its own (the matrix-core kernel)
constexpr uint32_t kHasTable = 1u << 24;
constexpr uint32_t kQuadPerGroup = 1u << 25;
inline uint32_t pack_heads(int kv_heads, int gq, bool has_table, bool quad_per_group = false) {
  return static_cast<uint32_t>(kv_heads) | (static_cast<uint32_t>(gq) << 16) | (has_table ? kHasTable : 0u) |
         (quad_per_group ? kQuadPerGroup : 0u);
}

// ---- split-K plan, shared by every kernel so the workspace size and the
// merge depend only on the shape, never on which kernel ran
struct SplitPlan {
  int splits;            // partitions of the attended blocks
  int blocks_per_split;  // consecutive attended blocks per partition
};
SplitPlan plan_splits(const kvssd_decode_desc& d, int units);

// ---- general kernel: any head_dim <= 256, group size, GQA ratio, block size
int launch_general(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts);

// ---- matrix-core kernel: head_dim 128, group_size 32, bits 2/4
bool mfma_supported(const kvssd_decode_desc& d, std::string* why);
bool mfma_aligned(const DecodeArgs& a);
int launch_mfma(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts);

// ---- LDS-staged matrix-core kernel: the matrix-core shapes with kv_heads % 4 == 0
bool staged_supported(const kvssd_decode_desc& d, std::string* why);
// whether the staged kernel takes 8 kv heads per workgroup for this shape
// (the split plan doubles its work items then)
bool staged_wide(const kvssd_decode_desc& d, int units);
bool staged_aligned(const DecodeArgs& a);
int launch_staged(const DecodeArgs& a, const SplitPlan& plan, SplitPartials parts);

// ---- split-K phase 2: merge the partials of every split into (out, lse);
// out holds elements of out_dtype (enum kvssd_dtype), lse fp32
int launch_merge_splits(SplitPartials parts, int splits, int query_heads, int head_dim, void* out, int out_dtype,
                        float* lse, hipStream_t stream);

// ---- chunk merge (pipeline), codec twins
int launch_merge_chunks(int rows, int dim, float* acc_out, float* acc_lse, const float* out, const float* lse,
                        hipStream_t stream);
// ---- record codec (records.hip)
int record_bytes_of(const kvssd_record_layout* layout, size_t* bytes);
int launch_gather_records(const kvssd_record_layout* layout, const uint8_t* records, size_t stride, int n,
                          int verify_crc, uint8_t* packed_k, uint8_t* packed_v, uint16_t* scales_k,
                          uint16_t* scales_v, int32_t* valid, int32_t* status, hipStream_t stream);
int launch_quantize(const void* x, int dtype, int64_t rows, int head_dim, int bits, int group_size, uint8_t* packed,
                    uint16_t* scales, hipStream_t stream);
int launch_encode_records(const kvssd_record_layout* layout, int dtype, const void* keys, const void* values,
                          int64_t tokens, int layer, int first_block, uint8_t* records, uint32_t* crcs,
                          hipStream_t stream);
// ---- vLLM block codec (vllm_codec.hip)
int vllm_sizes(int64_t elements, int bits, int group_size, size_t* record_bytes, size_t* scratch_bytes);
int launch_vllm_encode(const void* values, int dtype, int64_t elements, int bits, int group_size, uint8_t* record,
                       uint32_t* crc, void* scratch, size_t scratch_bytes, hipStream_t stream);
int launch_vllm_decode(const uint8_t* payload, int64_t elements, int bits, int group_size, uint32_t expected_crc,
                       int dtype, void* destination, int32_t* status, void* scratch, size_t scratch_bytes,
                       hipStream_t stream);
int launch_unpack_codes(const uint8_t* packed, int bits, int64_t n_bytes, uint8_t* codes, hipStream_t stream);
// ---- measurement: a plain streaming read (codec.hip)
size_t read_probe_sink_words();
int launch_read_probe(const void* data, size_t bytes, uint32_t* sink, hipStream_t stream);
int launch_dequantize(const uint8_t* packed, const uint16_t* scales, int64_t rows, int head_dim, int bits,
                      int group_size, float* out, hipStream_t stream);

}  // namespace kvssd
