// extern "C" entry points of libkvssd_hip.so (declared in include/kvssd_hip.h).
//
// Argument checks mirror the reference's (csrc/bindings.cpp:26-38,
// csrc/fused_decode.cu:117-121, src/kvssd/backends/base.py:29-55) so callers
// see the same failures; they run on the host before any launch, and every
// launch's grid is derived from the validated shape.
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "decode.hpp"

namespace kvssd {

namespace {
thread_local std::string g_last_error;

constexpr int kMaxDevices = 64;
std::once_flag g_props_once[kMaxDevices];
int g_is_gfx950[kMaxDevices];
char g_arch[kMaxDevices][64];

}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

int arg_error(const std::string& msg) {
  set_error(msg);
  return kArgError;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return 0;
  set_error(std::string(what) + ": " + hipGetErrorString(err));
  return static_cast<int>(err);
}

namespace {

int validate(const kvssd_decode_desc* d, int* units) {
  if (d == nullptr) return arg_error("descriptor is NULL");
  if (d->query_heads <= 0 || d->head_dim <= 0) return arg_error("query must be [query_heads, head_dim]");
  if (d->num_blocks <= 0 || d->block_tokens <= 0 || d->kv_heads <= 0)
    return arg_error("packed KV must match [blocks,tokens,kv_heads,packed_dim]");
  if (d->bits != 2 && d->bits != 4) return arg_error("bits must be 2 or 4");
  if (d->group_size <= 0 || d->head_dim % d->group_size) return arg_error("group_size must divide head_dim");
  if ((d->head_dim * d->bits) % 8) return arg_error("packed dimension does not match query head dimension");
  if (d->group_size % (8 / d->bits)) return arg_error("group_size must be positive and pack-aligned");
  if (d->query_heads % d->kv_heads) return arg_error("query heads must be divisible by KV heads");
  if (d->head_dim > 256) return arg_error("head_dim must be <= 256");
  if (d->query_dtype < KVSSD_DTYPE_F16 || d->query_dtype > KVSSD_DTYPE_F64) return arg_error("unsupported query dtype");
  if (d->kernel < KVSSD_KERNEL_AUTO || d->kernel > KVSSD_KERNEL_STAGED) return arg_error("unknown kernel selector");
  if (d->num_selected < 0) return arg_error("num_selected must be >= 0");
  if (d->out_query_dtype != 0 && d->out_query_dtype != 1) return arg_error("out_query_dtype must be 0 or 1");
  *units = d->num_blocks;
  return 0;
}

// Under AUTO, decodes of at most this many (kv head, attended block) pairs
// take the matrix-core kernel even where the staged one fits: its one-wave
// workgroups spread them over every CU, while the staged kernel (4 kv heads a
// workgroup below 2048 pairs) leaves most CUs idle.  Measured per step, 4K
// tokens: 8.7 against 9.7 us (GQA 4), 10.7 against 11.4 us (GQA 8); GQA 8
// with a 33-block table: 11.6 against 12.4 us; the two are even near 512
// pairs and the staged kernel wins from ~768 on.  At this size the
// matrix-core kernel gives each query quad of a kv head a workgroup of its
// own (GQA 8, split kernel: 4K 8.0 -> 7.1 us, the 33-block table 9.0 -> 8.0
// us), so its two-quad form -- which spills registers with a two-part fp32 /
// fp64 query -- never runs here (fp32 GQA 8: 7.8 against the staged kernel's
// 10.0 us).
constexpr long kSmallPairs = 512;

// Kernel for a shape (pointer alignment can still demote STAGED -> MFMA ->
// GENERAL under AUTO, see kvssd_hip_decode_partials).
int choose_kernel(const kvssd_decode_desc& d, int* kernel) {
  std::string why_mfma, why_staged;
  const bool mfma = mfma_supported(d, &why_mfma);
  const bool staged = mfma && staged_supported(d, &why_staged);
  if (d.kernel == KVSSD_KERNEL_STAGED) {
    if (!mfma) return arg_error("staged matrix-core kernel does not support this shape: " + why_mfma);
    if (!staged) return arg_error("staged matrix-core kernel does not support this shape: " + why_staged);
    *kernel = KVSSD_KERNEL_STAGED;
  } else if (d.kernel == KVSSD_KERNEL_MFMA) {
    if (!mfma) return arg_error("matrix-core kernel does not support this shape: " + why_mfma);
    *kernel = KVSSD_KERNEL_MFMA;
  } else if (d.kernel == KVSSD_KERNEL_GENERAL) {
    *kernel = KVSSD_KERNEL_GENERAL;
  } else {
    const long units = d.num_selected > 0 ? d.num_selected : d.num_blocks;
    const bool small = units * d.kv_heads <= kSmallPairs;
    *kernel = staged && !small ? KVSSD_KERNEL_STAGED : mfma ? KVSSD_KERNEL_MFMA : KVSSD_KERNEL_GENERAL;
  }
  return 0;
}

// Blocks attended by a call.  num_selected is the block table's length: a
// table needs num_selected >= 1, and num_selected must be 0 without one.  The
// phases that take no table pointer (merge, workspace size) read the same
// count from the descriptor, so every entry point plans the same splits.
int units_of(const kvssd_decode_desc* d, const int32_t* table, int* units) {
  if (table != nullptr) {
    if (d->num_selected <= 0) return arg_error("at least one block is required");
    *units = d->num_selected;
  } else if (d->num_selected != 0) {
    return arg_error("num_selected must be 0 when block_table is NULL");
  }
  return 0;
}

// The attended-block count of a descriptor alone (no table pointer): the
// phases without one plan from it.
int units_of_desc(const kvssd_decode_desc* d, int* units) {
  if (d->num_selected < 0) return arg_error("num_selected must be >= 0");
  *units = d->num_selected > 0 ? d->num_selected : d->num_blocks;
  return 0;
}

// Validation, unit count, kernel choice and split plan shared by the phases.
int plan_checked(const kvssd_decode_desc* desc, int units, const void* workspace, size_t workspace_bytes, int* kernel,
                 int* splits) {
  if (int rc = choose_kernel(*desc, kernel)) return rc;
  *splits = plan_splits(*desc, units).splits;
  const size_t need = split_partial_bytes(*splits, desc->query_heads, desc->head_dim);
  if (workspace == nullptr || workspace_bytes < need)
    return arg_error("workspace too small: need " + std::to_string(need) + " bytes");
  return 0;
}

int prepare(const kvssd_decode_desc* desc, const int32_t* table, void* workspace, size_t workspace_bytes, int* units,
            int* kernel, int* splits) {
  if (int rc = validate(desc, units)) return rc;
  if (int rc = units_of(desc, table, units)) return rc;
  return plan_checked(desc, *units, workspace, workspace_bytes, kernel, splits);
}

// ------------------------------------------------ no-allocation decode ---
// Split partials of kvssd_hip_fused_decode_static live in this file-scope
// device array instead of a caller's workspace.  Each GPU the library runs on
// holds its own copy (at its own address) until the process ends.  Host code
// never passes the array's name to a kernel or a copy: `scratch` is a
// host-side stand-in there; the device address comes from
// hipGetSymbolAddress, once per device with that device current.  Nothing in
// it has to start at zero: every split writes its whole partial before the
// merge reads it.  Calls that overlap on one GPU share the array and race.
constexpr size_t kStaticScratchBytes = size_t{16} << 20;  // 16 MiB
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

int static_scratch(void** ptr) {
  int dev = 0;
  if (hipError_t err = hipGetDevice(&dev); err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return arg_error("HIP device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); err != hipSuccess)
      return hip_status(err, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return hip_status(hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}

// Element type of `out`: fp32, or the query's dtype when the caller asks.
int out_dtype_of(const kvssd_decode_desc& d) { return d.out_query_dtype ? d.query_dtype : KVSSD_DTYPE_F32; }

// Both decode entry points: the split kernel, then (with `out`) the merge.
int decode_call(const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k, const uint8_t* packed_v,
                const uint16_t* scales_k, const uint16_t* scales_v, const int32_t* valid_tokens,
                const int32_t* block_table, void* workspace, size_t workspace_bytes, void* out, float* lse,
                void* stream) {
  int units = 0, kernel = 0, splits = 0;
  if (int rc = prepare(desc, block_table, workspace, workspace_bytes, &units, &kernel, &splits)) return rc;
  if (!query || !packed_k || !packed_v || !scales_k || !scales_v || !valid_tokens)
    return arg_error("a required buffer pointer is NULL");
  DecodeArgs a{};
  a.desc = *desc;
  a.query = query;
  a.packed_k = packed_k;
  a.packed_v = packed_v;
  a.scales_k = scales_k;
  a.scales_v = scales_v;
  a.valid = valid_tokens;
  a.table = block_table;
  a.units = units;
  a.stream = static_cast<hipStream_t>(stream);
  SplitPartials parts = carve_partials(workspace, splits, desc->query_heads, desc->head_dim);
  const SplitPlan plan = plan_splits(*desc, units);
  if (kernel == KVSSD_KERNEL_STAGED && !staged_aligned(a)) {
    if (desc->kernel == KVSSD_KERNEL_STAGED)
      return arg_error("staged matrix-core kernel needs 16-byte aligned packed arrays and scales");
    kernel = KVSSD_KERNEL_MFMA;
  }
  if (kernel == KVSSD_KERNEL_MFMA && !mfma_aligned(a)) {
    if (desc->kernel == KVSSD_KERNEL_MFMA)
      return arg_error(
          "matrix-core kernel needs 16-byte aligned packed arrays (8-byte for INT2) and 8-byte aligned scales");
    kernel = KVSSD_KERNEL_GENERAL;
  }
  int rc = kernel == KVSSD_KERNEL_STAGED ? launch_staged(a, plan, parts)
           : kernel == KVSSD_KERNEL_MFMA ? launch_mfma(a, plan, parts)
                                         : launch_general(a, plan, parts);
  if (rc != 0 || out == nullptr) return rc;
  return launch_merge_splits(parts, splits, desc->query_heads, desc->head_dim, out, out_dtype_of(*desc), lse,
                             a.stream);
}

}  // namespace
}  // namespace kvssd

using namespace kvssd;

extern "C" {

__attribute__((visibility("default"))) int kvssd_hip_abi_version(void) { return KVSSD_HIP_ABI_VERSION; }

// KVSSD_BUILD_ID comes from build.py (a hash of the sources and flags); the
// marked copy lets a loader find it in the file without mapping the library
#ifndef KVSSD_BUILD_ID
#define KVSSD_BUILD_ID "unknown"
#endif
__attribute__((used)) static const char kBuildIdMarked[] = "kvssd-build-id:" KVSSD_BUILD_ID;

__attribute__((visibility("default"))) const char* kvssd_hip_build_id(void) {
  return kBuildIdMarked + sizeof("kvssd-build-id:") - 1;
}

__attribute__((visibility("default"))) const char* kvssd_hip_last_error(void) { return g_last_error.c_str(); }

__attribute__((visibility("default"))) int kvssd_hip_device_ok(int device, char* why, size_t why_len) {
  auto say = [&](const std::string& s) {
    if (why != nullptr && why_len > 0) {
      std::snprintf(why, why_len, "%s", s.c_str());
    }
  };
  int count = 0;
  hipError_t err = hipGetDeviceCount(&count);
  if (err != hipSuccess || count <= 0) {
    say("no HIP device is visible");
    return 0;
  }
  if (device < 0 || device >= count || device >= kMaxDevices) {
    say("HIP device index out of range");
    return 0;
  }
  std::call_once(g_props_once[device], [device] {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
      std::snprintf(g_arch[device], sizeof(g_arch[device]), "%s", prop.gcnArchName);
      g_is_gfx950[device] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    } else {
      std::snprintf(g_arch[device], sizeof(g_arch[device]), "%s", "unknown");
      g_is_gfx950[device] = 0;
    }
  });
  if (!g_is_gfx950[device]) {
    say("libkvssd_hip is built for gfx950 (MI355X); device " + std::to_string(device) + " is " + std::string(g_arch[device]));
    return 0;
  }
  say("gfx950 HIP kernels available");
  return 1;
}

__attribute__((visibility("default"))) int kvssd_hip_decode_kernel(const kvssd_decode_desc* desc, int* kernel) {
  int units = 0;
  if (int rc = validate(desc, &units)) return rc;
  if (kernel == nullptr) return arg_error("kernel output pointer is NULL");
  return choose_kernel(*desc, kernel);
}

__attribute__((visibility("default"))) int kvssd_hip_decode_workspace_bytes(const kvssd_decode_desc* desc,
                                                                            size_t* bytes) {
  int units = 0;
  if (int rc = validate(desc, &units)) return rc;
  if (bytes == nullptr) return arg_error("bytes output pointer is NULL");
  if (int rc = units_of_desc(desc, &units)) return rc;
  int kernel = 0;
  if (int rc = choose_kernel(*desc, &kernel)) return rc;
  *bytes = split_partial_bytes(plan_splits(*desc, units).splits, desc->query_heads, desc->head_dim);
  return 0;
}

__attribute__((visibility("default"))) int kvssd_hip_decode_partials(
    const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k, const uint8_t* packed_v,
    const uint16_t* scales_k, const uint16_t* scales_v, const int32_t* valid_tokens, const int32_t* block_table,
    void* workspace, size_t workspace_bytes, void* stream) {
  return decode_call(desc, query, packed_k, packed_v, scales_k, scales_v, valid_tokens, block_table, workspace,
                     workspace_bytes, nullptr, nullptr, stream);
}

__attribute__((visibility("default"))) int kvssd_hip_decode_merge(const kvssd_decode_desc* desc,
                                                                  const void* workspace, size_t workspace_bytes,
                                                                  void* out, float* lse, void* stream) {
  int units = 0, kernel = 0, splits = 0;
  if (int rc = validate(desc, &units)) return rc;
  if (int rc = units_of_desc(desc, &units)) return rc;
  if (int rc = plan_checked(desc, units, workspace, workspace_bytes, &kernel, &splits)) return rc;
  if (!out || !lse) return arg_error("a required buffer pointer is NULL");
  SplitPartials parts = carve_partials(const_cast<void*>(workspace), splits, desc->query_heads, desc->head_dim);
  return launch_merge_splits(parts, splits, desc->query_heads, desc->head_dim, out, out_dtype_of(*desc), lse,
                             static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_fused_decode(
    const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k, const uint8_t* packed_v,
    const uint16_t* scales_k, const uint16_t* scales_v, const int32_t* valid_tokens, const int32_t* block_table,
    void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  if (!out || !lse) return arg_error("a required buffer pointer is NULL");
  return decode_call(desc, query, packed_k, packed_v, scales_k, scales_v, valid_tokens, block_table, workspace,
                     workspace_bytes, out, lse, stream);
}

__attribute__((visibility("default"))) int kvssd_hip_fused_decode_static(
    const kvssd_decode_desc* desc, const void* query, const uint8_t* packed_k, const uint8_t* packed_v,
    const uint16_t* scales_k, const uint16_t* scales_v, const int32_t* valid_tokens, const int32_t* block_table,
    void* out, float* lse, void* stream) {
  if (!out || !lse) return arg_error("a required buffer pointer is NULL");
  size_t need = 0;
  if (int rc = kvssd_hip_decode_workspace_bytes(desc, &need)) return rc;
  if (need > kStaticScratchBytes)
    return arg_error("this shape needs " + std::to_string(need) + " bytes of split partials, more than the " +
                     std::to_string(kStaticScratchBytes) +
                     "-byte static scratch; use kvssd_hip_fused_decode with a workspace");
  void* ptr = nullptr;
  if (int rc = static_scratch(&ptr)) return rc;
  return decode_call(desc, query, packed_k, packed_v, scales_k, scales_v, valid_tokens, block_table, ptr,
                     kStaticScratchBytes, out, lse, stream);
}

__attribute__((visibility("default"))) int kvssd_hip_merge_chunks(int rows, int dim, float* acc_out, float* acc_lse,
                                                                  const float* out, const float* lse, void* stream) {
  if (rows <= 0 || dim <= 0) return arg_error("merge needs positive rows and dim");
  if (!acc_out || !acc_lse || !out || !lse) return arg_error("a required buffer pointer is NULL");
  return launch_merge_chunks(rows, dim, acc_out, acc_lse, out, lse, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_unpack_codes(const uint8_t* packed, int bits, int64_t n_bytes,
                                                                  uint8_t* codes, void* stream) {
  if (bits != 2 && bits != 4) return arg_error("bits must be 2 or 4");
  if (n_bytes < 0) return arg_error("n_bytes must be non-negative");
  if (n_bytes > 0 && (!packed || !codes)) return arg_error("a required buffer pointer is NULL");
  return launch_unpack_codes(packed, bits, n_bytes, codes, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_dequantize(const uint8_t* packed, const uint16_t* scales,
                                                                int64_t rows, int head_dim, int bits, int group_size,
                                                                float* out, void* stream) {
  if (bits != 2 && bits != 4) return arg_error("bits must be 2 or 4");
  if (rows < 0 || head_dim <= 0) return arg_error("rows must be >= 0 and head_dim positive");
  if (group_size <= 0 || head_dim % group_size) return arg_error("group_size must divide head_dim");
  if ((head_dim * bits) % 8) return arg_error("packed dimension does not match query head dimension");
  if (rows > 0 && (!packed || !scales || !out)) return arg_error("a required buffer pointer is NULL");
  return launch_dequantize(packed, scales, rows, head_dim, bits, group_size, out, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_record_bytes(const kvssd_record_layout* layout, size_t* bytes) {
  return record_bytes_of(layout, bytes);
}

__attribute__((visibility("default"))) int kvssd_hip_gather_records(
    const kvssd_record_layout* layout, const uint8_t* records, size_t stride, int n, int verify_crc,
    uint8_t* packed_k, uint8_t* packed_v, uint16_t* scales_k, uint16_t* scales_v, int32_t* valid, int32_t* status,
    void* stream) {
  return launch_gather_records(layout, records, stride, n, verify_crc, packed_k, packed_v, scales_k, scales_v, valid,
                               status, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_quantize(const void* x, int dtype, int64_t rows, int head_dim,
                                                              int bits, int group_size, uint8_t* packed,
                                                              uint16_t* scales, void* stream) {
  return launch_quantize(x, dtype, rows, head_dim, bits, group_size, packed, scales,
                         static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_encode_records(const kvssd_record_layout* layout, int dtype,
                                                                    const void* keys, const void* values,
                                                                    int64_t tokens, int layer, int first_block,
                                                                    uint8_t* records, uint32_t* crcs, void* stream) {
  return launch_encode_records(layout, dtype, keys, values, tokens, layer, first_block, records, crcs,
                               static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_vllm_sizes(int64_t elements, int bits, int group_size,
                                                                size_t* record_bytes, size_t* scratch_bytes) {
  return vllm_sizes(elements, bits, group_size, record_bytes, scratch_bytes);
}

__attribute__((visibility("default"))) int kvssd_hip_vllm_encode(const void* values, int dtype, int64_t elements,
                                                                 int bits, int group_size, uint8_t* record,
                                                                 uint32_t* crc, void* scratch, size_t scratch_bytes,
                                                                 void* stream) {
  return launch_vllm_encode(values, dtype, elements, bits, group_size, record, crc, scratch, scratch_bytes,
                            static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_vllm_decode(const uint8_t* payload, int64_t elements, int bits,
                                                                 int group_size, uint32_t crc, int dtype,
                                                                 void* destination, int32_t* status, void* scratch,
                                                                 size_t scratch_bytes, void* stream) {
  return launch_vllm_decode(payload, elements, bits, group_size, crc, dtype, destination, status, scratch,
                            scratch_bytes, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_read_probe(const void* data, size_t bytes, uint32_t* sink,
                                                                size_t sink_words, void* stream) {
  if (bytes % 16) return arg_error("read probe bytes must be a multiple of 16");
  if (bytes > 0 && (!data || !sink)) return arg_error("a required buffer pointer is NULL");
  if ((reinterpret_cast<uintptr_t>(data) % 16) != 0) return arg_error("read probe data must be 16-byte aligned");
  if (sink_words < read_probe_sink_words())
    return arg_error("read probe sink needs " + std::to_string(read_probe_sink_words()) + " words");
  return launch_read_probe(data, bytes, sink, static_cast<hipStream_t>(stream));
}

__attribute__((visibility("default"))) int kvssd_hip_memcpy_h2d_async(void* dst, const void* src, size_t bytes,
                                                                      void* stream) {
  if (bytes == 0) return 0;
  if (!dst || !src) return arg_error("a required buffer pointer is NULL");
  return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)),
                    "hipMemcpyAsync");
}

}  // extern "C"
