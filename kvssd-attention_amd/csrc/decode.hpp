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
  float* out;
  float* lse;
  hipStream_t stream;
};

// ---- general kernel: any head_dim <= 256, group size, GQA ratio, block size
struct GeneralPlan {
  int splits;           // token-axis splits (grid.x)
  int blocks_per_split; // consecutive units per split
  int heads_per_chunk;  // query heads per workgroup (<= 8)
  int head_chunks;      // workgroups per kv head along the query-head axis
};
GeneralPlan plan_general(const kvssd_decode_desc& d, int units);
int launch_general(const DecodeArgs& a, const GeneralPlan& plan, SplitPartials parts);

// ---- matrix-core kernel: head_dim 128, group_size 32, bits 2/4
struct MfmaPlan {
  int splits;           // waves per kv head along the token axis
  int blocks_per_split; // units per wave
  int head_quads;       // groups of 4 query heads per kv head
};
bool mfma_supported(const kvssd_decode_desc& d, std::string* why);
MfmaPlan plan_mfma(const kvssd_decode_desc& d, int units);
int launch_mfma(const DecodeArgs& a, const MfmaPlan& plan, SplitPartials parts);

// ---- split-K phase 2: merge the partials of every split into (out, lse)
int launch_merge_splits(SplitPartials parts, int splits, int query_heads, int head_dim, float* out, float* lse,
                        hipStream_t stream);

// ---- chunk merge (pipeline), codec twins
int launch_merge_chunks(int rows, int dim, float* acc_out, float* acc_lse, const float* out, const float* lse,
                        hipStream_t stream);
int launch_unpack_codes(const uint8_t* packed, int bits, int64_t n_bytes, uint8_t* codes, hipStream_t stream);
int launch_dequantize(const uint8_t* packed, const uint16_t* scales, int64_t rows, int head_dim, int bits,
                      int group_size, float* out, hipStream_t stream);

}  // namespace kvssd
