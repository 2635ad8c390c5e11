/*
 * kvssd_hip.h: C ABI of libkvssd_hip.so, the MI355X (gfx950) fused INT2/INT4
 * dequant + decode-attention library.
 *
 * This ABI replaces the reference's pybind/torch extension kvssd._C
 * (csrc/bindings.cpp:16-45, csrc/fused_decode.cu:92-143).  It uses plain C
 * types only: device pointers, sizes and a hipStream_t passed as void*.
 *
 * Conventions
 *   - Every call returns 0 on success.  A negative value is an argument error:
 *     the message is available from kvssd_hip_last_error() and mirrors the
 *     reference's check (the Python layer raises ValueError).  A positive value
 *     is a hipError_t from the runtime (the Python layer raises RuntimeError).
 *   - The caller allocates every buffer, including the workspace.  The library
 *     never allocates or frees device memory.
 *   - Every launch is asynchronous on `stream` (a hipStream_t; NULL means the
 *     null stream); no call synchronises the host.
 *   - The library keeps no per-call state; the only global state is a
 *     thread-local error string and a per-device property cache filled once.
 *     Calls are reentrant from any host thread.
 */
#ifndef KVSSD_HIP_H
#define KVSSD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVSSD_HIP_ABI_VERSION 5

/* Query element types accepted by kvssd_hip_fused_decode (the reference
 * dispatches fp32/fp64/fp16/bf16 queries: csrc/fused_decode.cu:131-133). */
enum kvssd_dtype {
  KVSSD_DTYPE_F16 = 0,
  KVSSD_DTYPE_BF16 = 1,
  KVSSD_DTYPE_F32 = 2,
  KVSSD_DTYPE_F64 = 3
};

/* Kernel selection for kvssd_hip_fused_decode. */
enum kvssd_kernel {
  KVSSD_KERNEL_AUTO = 0,    /* fastest kernel that supports the shape */
  KVSSD_KERNEL_GENERAL = 1, /* any shape the reference accepts */
  KVSSD_KERNEL_MFMA = 2,    /* matrix-core kernel: head_dim 128, group_size 32 */
  KVSSD_KERNEL_STAGED = 3   /* LDS-staged matrix-core kernel: as MFMA, plus
                               kv_heads % 4 == 0 and 16-byte aligned arrays */
};

/* Shape of one decode call.  The packed arrays follow the reference's
 * PackedBatch layout (src/kvssd/backends/base.py:19-27):
 *   packed_k, packed_v  uint8   [num_blocks, block_tokens, kv_heads, head_dim*bits/8]
 *   scales_k, scales_v  float16 [num_blocks, block_tokens, kv_heads, head_dim/group_size]
 *   valid_tokens        int32   [num_blocks]
 * all C-contiguous.  When block_table is not NULL it lists num_selected >= 1
 * block ids (int32, each in [0, num_blocks)) and the call attends over those
 * blocks in table order; with NULL, num_selected must be 0 and the call attends
 * over blocks 0..num_blocks-1.  The entry points without a table argument
 * (kvssd_hip_decode_workspace_bytes, kvssd_hip_decode_kernel,
 * kvssd_hip_decode_merge) plan for num_selected blocks when it is > 0, else for
 * num_blocks, so they agree with the call that passes the table. */
typedef struct kvssd_decode_desc {
  int32_t query_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t num_blocks;
  int32_t block_tokens;
  int32_t bits;
  int32_t group_size;
  int32_t query_dtype;  /* enum kvssd_dtype */
  int32_t num_selected; /* entries in block_table; 0 when there is none */
  int32_t kernel;       /* enum kvssd_kernel */
  double sm_scale;
  int32_t out_query_dtype; /* 0: out is fp32 (the reference's output);
                              1: out holds query_dtype elements, each the
                              fp32 result rounded to nearest even (what the
                              reference's pipeline does next with
                              .to(query.dtype), src/kvssd/pipeline.py:165);
                              lse is fp32 either way */
} kvssd_decode_desc;

/* ABI version of the loaded library (KVSSD_HIP_ABI_VERSION). */
int kvssd_hip_abi_version(void);

/* The build's identity: a hash of the HIP sources, this header and the
 * compile flags the library was built from, as a NUL-terminated hex string
 * (no counterpart in the reference, which JIT-builds its extension; the
 * Python layer compares it with the tree's sources and refuses a stale
 * build). */
const char* kvssd_hip_build_id(void);

/* 1 when `device` is a gfx950 GPU this library has code for, else 0, with the
 * reason written to `why` (NUL-terminated, at most why_len bytes).  Backs
 * HipAttentionBackend.probe(); replaces the device check of
 * src/kvssd/backends/cuda.py:20-29. */
int kvssd_hip_device_ok(int device, char* why, size_t why_len);

/* Device workspace bytes kvssd_hip_fused_decode needs for `desc`. */
int kvssd_hip_decode_workspace_bytes(const kvssd_decode_desc* desc, size_t* bytes);

/* Which kernel kvssd_hip_fused_decode would run for `desc` (enum kvssd_kernel;
 * never KVSSD_KERNEL_AUTO). */
int kvssd_hip_decode_kernel(const kvssd_decode_desc* desc, int* kernel);

/* Fused decode attention over a packed batch: out [query_heads, head_dim]
 * (softmax-normalised; fp32, or query_dtype with desc->out_query_dtype = 1),
 * lse fp32 [query_heads] (natural-log log-sum-exp of the
 * scaled scores).  Replaces kvssd._C.fused_decode (csrc/bindings.cpp:16-41,
 * csrc/fused_decode.cu:92-143) with the semantics of
 * ReferenceAttentionBackend.run (src/kvssd/backends/reference.py:22-50):
 * block b contributes the rows keys[b, :valid_tokens[b]] would keep in Python
 * (reference.py:38-40): min(v, block_tokens) rows for v >= 0 and
 * max(block_tokens + v, 0) rows for v < 0.  With no valid token at all out is
 * 0 and lse is -inf.  `query` holds query_heads*head_dim elements of
 * query_dtype. */
int kvssd_hip_fused_decode(const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k,
                           const uint8_t* packed_v, const uint16_t* scales_k, const uint16_t* scales_v,
                           const int32_t* valid_tokens, const int32_t* block_table, void* out, float* lse,
                           void* workspace, size_t workspace_bytes, void* stream);

/* kvssd_hip_fused_decode with no workspace argument and no allocation: the
 * split partials go to a 16 MiB array of device memory the library holds per
 * GPU for the life of the process.  No counterpart in the reference; it is
 * for callers that cannot allocate device memory (HIP graph capture, serving
 * loops that forbid it).  Shapes whose partials need more than 16 MiB (see
 * kvssd_hip_decode_workspace_bytes) fail with an argument error.  Calls that
 * overlap on one GPU share the array and race: issue them on one stream (or
 * order them) per GPU. */
int kvssd_hip_fused_decode_static(const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k,
                                  const uint8_t* packed_v, const uint16_t* scales_k, const uint16_t* scales_v,
                                  const int32_t* valid_tokens, const int32_t* block_table, void* out, float* lse,
                                  void* stream);

/* Phase 1 of kvssd_hip_fused_decode alone: every split writes its
 * unnormalised partial (O, running max, running sum) into `workspace`.
 * kvssd_hip_decode_merge turns them into (out, lse).  Same arguments and checks
 * as kvssd_hip_fused_decode; no reference counterpart (the reference kernel is
 * one pass, csrc/fused_decode.cu:12-90).  Lets a caller time or overlap the
 * two phases separately. */
int kvssd_hip_decode_partials(const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k,
                              const uint8_t* packed_v, const uint16_t* scales_k, const uint16_t* scales_v,
                              const int32_t* valid_tokens, const int32_t* block_table, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Phase 2: merge the split partials left in `workspace` by
 * kvssd_hip_decode_partials for the same `desc` into out / lse. */
int kvssd_hip_decode_merge(const kvssd_decode_desc* desc, const void* workspace, size_t workspace_bytes, void* out,
                           float* lse, void* stream);

/* Running exact merge of normalised attention chunks, in place:
 *   L = logaddexp(acc_lse, lse); acc_out = acc_out e^(acc_lse-L) + out e^(lse-L)
 * over `rows` rows of `dim` fp32 values.  Replaces merge_attention_chunks
 * (src/kvssd/attention.py:91-102) in the pipeline's chunk loop
 * (src/kvssd/pipeline.py:147-153).  A chunk with lse = -inf adds nothing. */
int kvssd_hip_merge_chunks(int rows, int dim, float* acc_out, float* acc_lse, const float* out, const float* lse,
                           void* stream);

/* Unsigned codes of `n_bytes` packed bytes (8/bits codes per byte, low bits
 * first), unpacked by the same in-register routine the fused kernels use.
 * Bit-exact twin of unpack_codes (src/kvssd/quant.py:40-46). */
int kvssd_hip_unpack_codes(const uint8_t* packed, int bits, int64_t n_bytes, uint8_t* codes, void* stream);

/* fp32 (code - mid) * scale for `rows` rows of `head_dim` elements
 * (packed [rows, head_dim*bits/8], scales [rows, head_dim/group_size]).
 * Twin of dequantize_tensor (src/kvssd/quant.py:68-73); exact. */
int kvssd_hip_dequantize(const uint8_t* packed, const uint16_t* scales, int64_t rows, int head_dim, int bits,
                         int group_size, float* out, void* stream);

/* Shape of a v1 KV block record: the CacheSpec fields that lay it out
 * (src/kvssd/format.py:23-58). */
typedef struct kvssd_record_layout {
  int32_t bits;
  int32_t block_tokens;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t group_size;
} kvssd_record_layout;

/* Bytes of one record: the 52-byte header plus the payload, padded to a 4096
 * multiple (CacheSpec.record_bytes, src/kvssd/format.py:53-58). */
int kvssd_hip_record_bytes(const kvssd_record_layout* layout, size_t* bytes);

/* `n` raw records in device memory, `stride` bytes apart (4-byte aligned),
 * into the PackedBatch arrays: packed_k/v [n, BT, KVH, PD], scales_k/v fp16
 * [n, BT, KVH, G], valid [n] (the header's valid tokens), and status [n]:
 * 0 ok, 1 invalid header (magic or version), 2 layout differs from `layout`,
 * 3 payload length or CRC-32 mismatch (checked when verify_crc != 0).
 * The GPU form of decode_record (src/kvssd/format.py:134-177) over a span of
 * records, replacing the loader's payload clones and the pipeline's per-array
 * stacking (src/kvssd/loader.py:73-91, src/kvssd/pipeline.py:98-108). */
int kvssd_hip_gather_records(const kvssd_record_layout* layout, const uint8_t* records, size_t stride, int n,
                             int verify_crc, uint8_t* packed_k, uint8_t* packed_v, uint16_t* scales_k,
                             uint16_t* scales_v, int32_t* valid, int32_t* status, void* stream);

/* Groupwise quantisation of `rows` rows of `head_dim` values of `dtype`
 * (kvssd_dtype): packed [rows, head_dim*bits/8] (low bits first), fp16 scales
 * [rows, head_dim/group_size].  Bit-exact twin of quantize_tensor
 * (src/kvssd/quant.py:49-65). */
int kvssd_hip_quantize(const void* x, int dtype, int64_t rows, int head_dim, int bits, int group_size,
                       uint8_t* packed, uint16_t* scales, void* stream);

/* Records of one layer: keys and values [tokens, KVH, D] of `dtype` become
 * ceil(tokens / BT) records (record_bytes each) for blocks first_block,
 * first_block + 1, ... -- the last block zero-padded -- and their payload
 * CRC-32 in crcs.  KVCacheStore.create's block loop (src/kvssd/store.py:46-63)
 * with encode_record (src/kvssd/format.py:104-131), on the GPU. */
int kvssd_hip_encode_records(const kvssd_record_layout* layout, int dtype, const void* keys, const void* values,
                             int64_t tokens, int layer, int first_block, uint8_t* records, uint32_t* crcs,
                             void* stream);

/* vLLM block records (src/kvssd/integrations/vllm_codec.py:18-102): a 32-byte
 * header "<8sBBBBIIQI" ("KVVLLM02", version 1, bits, dtype code 1/2/3 for
 * float16/bfloat16/float32, 0, group_size, elements, payload bytes, CRC-32),
 * payload = fp16 scales [elements / group_size] | codes [elements * bits / 8]
 * of the block's values as one flat vector, zero padding to a 4096 multiple.
 * Record size and the device scratch bytes kvssd_hip_vllm_encode / _decode
 * need for a block of `elements` values (payload at most 16 MiB). */
int kvssd_hip_vllm_sizes(int64_t elements, int bits, int group_size, size_t* record_bytes, size_t* scratch_bytes);

/* encode_vllm_block (vllm_codec.py:42-70) on the GPU: `elements` values of
 * `dtype` (F16, BF16 or F32) -> the whole record at `record` (4-byte aligned,
 * kvssd_hip_vllm_sizes bytes) and its payload CRC-32 in *crc (device). */
int kvssd_hip_vllm_encode(const void* values, int dtype, int64_t elements, int bits, int group_size, uint8_t* record,
                          uint32_t* crc, void* scratch, size_t scratch_bytes, void* stream);

/* The GPU half of decode_vllm_block (vllm_codec.py:73-102): the caller has
 * parsed and checked the header (magic, version, dtype, payload length); this
 * verifies the payload CRC-32 against `crc` (*status = 0, or 3 on a mismatch)
 * and dequantises the codes into `destination` (`elements` values of `dtype`),
 * (code - mid) * scale in fp32 rounded once, as dequantize_tensor(q, dtype). */
int kvssd_hip_vllm_decode(const uint8_t* payload, int64_t elements, int bits, int group_size, uint32_t crc, int dtype,
                          void* destination, int32_t* status, void* scratch, size_t scratch_bytes, void* stream);

/* Plain streaming read of `bytes` bytes at `data` (16-byte aligned, a
 * multiple of 16), XOR-folded into `sink` (at least 8,192 dwords).  A
 * measurement helper with no counterpart in the reference: the HBM read rate
 * a plain kernel attains on this GPU, which the decode's packed-KV rate is
 * compared with. */
int kvssd_hip_read_probe(const void* data, size_t bytes, uint32_t* sink, size_t sink_words, void* stream);

/* hipMemcpyAsync host->device of `bytes` bytes on `stream`; `src` should be
 * page-locked for the copy to be asynchronous.  The staging copy of
 * KVSSDPipeline._stage (src/kvssd/pipeline.py:110-114). */
int kvssd_hip_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream);

/* Message of the last failed call on this host thread ("" if none). */
const char* kvssd_hip_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KVSSD_HIP_H */
