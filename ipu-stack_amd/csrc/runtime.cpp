// libipus host runtime: context, buffers, events, the kernel ABI registry and
// ipus_launch, synthetic input generation.  C ABI in include/ipus.h.
#include "../../include/ipus.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cctype>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "internal.h"
#include "kernels.h"

namespace ipus {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* fmt, ...) {
  char buffer[1024];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error = buffer;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(IPUS_ERROR_HIP_BASE - (int)e, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// Makes the context's device current for the calling thread.
int use_device(const ipus_context* ctx) {
  const hipError_t e = hipSetDevice(ctx->device);
  return e == hipSuccess ? 0 : hip_fail(e, "hipSetDevice");
}

int check_launch(int status, const char* symbol) {
  if (status == 0) return 0;
  if (status <= IPUS_ERROR_HIP_BASE)
    return fail(status, "%s: launch failed: %s", symbol,
                hipGetErrorString((hipError_t)(IPUS_ERROR_HIP_BASE - status)));
  switch (status) {
    case IPUS_ERROR_UNAVAILABLE:
      return fail(status, "kernel %s has no device implementation for these arguments", symbol);
    case IPUS_ERROR_UNSUPPORTED_COUNT:
      return fail(status, "kernel %s does not support this element count", symbol);
    default:
      return fail(status, "kernel %s rejected its arguments", symbol);
  }
}

}  // namespace ipus

using namespace ipus;



// ---------------------------------------------------------------------------
// Errors, version
// ---------------------------------------------------------------------------
extern "C" const char* ipus_last_error(void) { return g_last_error.c_str(); }
extern "C" const char* ipus_version(void) { return "libipus 0.1.0 (gfx950)"; }

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
extern "C" int ipus_device_count(int* count) {
  if (!count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "count is null");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return 0;
  }
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  *count = n;
  return 0;
}

extern "C" int ipus_context_create(int device, ipus_context** out) {
  if (!out) return fail(IPUS_ERROR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return fail(IPUS_ERROR_NO_DEVICE, "no HIP device is available (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, n);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  auto* ctx = new ipus_context();
  ctx->device = device;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipStreamCreate");
  }
  // Per-device address of the no-allocation entry point's scratch array,
  // looked up once per device with that device current.
  if (int status = split_scratch_init(device)) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(status, "device %d: looking up the split-K scratch array failed (%d)", device,
                status);
  }
  *out = ctx;
  return 0;
}

extern "C" int ipus_context_destroy(ipus_context* ctx) {
  if (!ctx) return 0;
  // The context is released even when the device reports an error; the
  // first error is returned.
  int status = use_device(ctx);
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess && status == 0) status = hip_fail(e, "hipStreamSynchronize");
  e = hipStreamDestroy(ctx->stream);
  if (e != hipSuccess && status == 0) status = hip_fail(e, "hipStreamDestroy");
  // Buffers the caller did not free are released with the context.
  for (const auto& kv : ctx->live) {
    e = hipFree(kv.first);
    if (e != hipSuccess && status == 0) status = hip_fail(e, "hipFree");
  }
  delete ctx;
  return status;
}

namespace {
// Reads the first line of a text file into `out`; false if it is absent or
// empty.
bool read_line(const char* path, char* out, size_t size) {
  FILE* f = fopen(path, "r");
  if (!f) return false;
  const bool ok = fgets(out, (int)size, f) != nullptr;
  fclose(f);
  if (!ok) return false;
  out[strcspn(out, "\r\n")] = '\0';
  return out[0] != '\0';
}

// Where the runtime reports an empty device name: the product name the
// amdgpu driver exposes for the device's PCI function, else for the first
// card that has one, else the architecture and CU count.
void device_product_name(int device, const hipDeviceProp_t& p, char* out, size_t size) {
  char bus[64] = {0}, path[160];
  if (hipDeviceGetPCIBusId(bus, (int)sizeof(bus), device) == hipSuccess && bus[0]) {
    for (char* c = bus; *c; ++c) *c = (char)tolower((unsigned char)*c);
    snprintf(path, sizeof(path), "/sys/bus/pci/devices/%s/product_name", bus);
    if (read_line(path, out, size)) return;
  }
  for (int card = 0; card < 64; ++card) {
    snprintf(path, sizeof(path), "/sys/class/drm/card%d/device/product_name", card);
    if (read_line(path, out, size)) return;
  }
  char arch[32];
  snprintf(arch, sizeof(arch), "%s", p.gcnArchName);
  arch[strcspn(arch, ":")] = '\0';
  snprintf(out, size, "AMD GPU %s (%d CUs)", arch, p.multiProcessorCount);
}
}  // namespace

extern "C" int ipus_context_device_info(ipus_context* ctx, ipus_device_info* info) {
  if (!ctx || !info) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, ctx->device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  memset(info, 0, sizeof(*info));
  snprintf(info->name, sizeof(info->name), "%s", p.name);
  if (!info->name[0]) device_product_name(ctx->device, p, info->name, sizeof(info->name));
  snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
  info->compute_units = p.multiProcessorCount;
  info->clock_khz = p.clockRate;
  info->memory_clock_khz = p.memoryClockRate;
  info->memory_bus_width = p.memoryBusWidth;
  info->global_memory_bytes = p.totalGlobalMem;
  info->lds_bytes_per_block = (int)p.sharedMemPerBlock;
  return 0;
}

extern "C" int ipus_context_stream(ipus_context* ctx, void** stream) {
  if (!ctx || !stream) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  *stream = (void*)ctx->stream;
  return 0;
}

// ---------------------------------------------------------------------------
// Buffers
// ---------------------------------------------------------------------------
extern "C" int ipus_buffer_alloc(ipus_context* ctx, size_t bytes, void** ptr) {
  if (!ctx || !ptr) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (int e = use_device(ctx)) return e;
  // 256-byte aligned by hipMalloc; zero-byte requests get a valid pointer.
  hipError_t e = hipMalloc(ptr, bytes ? bytes : 256);
  if (e == hipErrorOutOfMemory)
    return fail(IPUS_ERROR_OUT_OF_MEMORY, "out of device memory allocating %zu bytes", bytes);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  std::lock_guard<std::mutex> lock(ctx->live_mutex);
  ctx->live[*ptr] = bytes;
  return 0;
}

extern "C" int ipus_buffer_free(ipus_context* ctx, void* ptr) {
  if (!ctx) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null context");
  if (!ptr) return 0;
  {
    std::lock_guard<std::mutex> lock(ctx->live_mutex);
    auto it = ctx->live.find(ptr);
    if (it == ctx->live.end())
      return fail(IPUS_ERROR_INVALID_ARGUMENT, "%p is not a live buffer of this context", ptr);
    ctx->live.erase(it);
  }
  if (int e = use_device(ctx)) return e;
  hipError_t e = hipFree(ptr);
  if (e != hipSuccess) return hip_fail(e, "hipFree");
  return 0;
}

extern "C" int ipus_context_live_buffers(ipus_context* ctx, uint64_t* count, uint64_t* bytes) {
  if (!ctx || !count || !bytes) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> lock(ctx->live_mutex);
  *count = ctx->live.size();
  uint64_t total = 0;
  for (const auto& kv : ctx->live) total += kv.second;
  *bytes = total;
  return 0;
}

extern "C" int ipus_context_inject_launch_failure(ipus_context* ctx, uint32_t launches_before,
                                                  int status) {
  if (!ctx) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null context");
  if (status > 0) return fail(IPUS_ERROR_INVALID_ARGUMENT, "injected status must be <= 0");
  ctx->inject_after = launches_before;
  ctx->inject_status = status;
  return 0;
}

extern "C" int ipus_buffer_upload(ipus_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes))
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (!bytes) return 0;
  if (int status = use_device(ctx)) return status;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "upload");
  return 0;
}

extern "C" int ipus_buffer_download(ipus_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes))
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (!bytes) return 0;
  if (int status = use_device(ctx)) return status;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "download");
  return 0;
}

extern "C" int ipus_buffer_copy(ipus_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes))
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (!bytes) return 0;
  if (int status = use_device(ctx)) return status;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "copy");
  return 0;
}

extern "C" int ipus_buffer_memset(ipus_context* ctx, void* ptr, int value, size_t bytes) {
  if (!ctx || (!ptr && bytes)) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (!bytes) return 0;
  if (int status = use_device(ctx)) return status;
  hipError_t e = hipMemsetAsync(ptr, value, bytes, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "memset");
  return 0;
}

// ---------------------------------------------------------------------------
// Sync and events
// ---------------------------------------------------------------------------
struct ipus_event {
  hipEvent_t event;
};

extern "C" int ipus_stream_sync(ipus_context* ctx) {
  if (!ctx) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null context");
  if (int status = use_device(ctx)) return status;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  return 0;
}

extern "C" int ipus_event_create(ipus_context* ctx, ipus_event** out) {
  if (!ctx || !out) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (int e = use_device(ctx)) return e;
  auto* ev = new ipus_event();
  hipError_t e = hipEventCreate(&ev->event);
  if (e != hipSuccess) {
    delete ev;
    return hip_fail(e, "hipEventCreate");
  }
  *out = ev;
  return 0;
}

extern "C" int ipus_event_destroy(ipus_event* ev) {
  if (!ev) return 0;
  const hipError_t e = hipEventDestroy(ev->event);
  delete ev;
  return e == hipSuccess ? 0 : hip_fail(e, "hipEventDestroy");
}

extern "C" int ipus_event_record(ipus_context* ctx, ipus_event* ev) {
  if (!ctx || !ev) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (int status = use_device(ctx)) return status;
  hipError_t e = hipEventRecord(ev->event, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  return 0;
}

extern "C" int ipus_event_elapsed_ms(ipus_event* start, ipus_event* end, float* ms) {
  if (!start || !end || !ms) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  hipError_t e = hipEventSynchronize(end->event);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, start->event, end->event);
  if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
  return 0;
}

// ---------------------------------------------------------------------------
// Kernel ABI registry and launch (tile_kernel_abi / validate_kernel_run /
// ComputeStep, crates/ipu-codegen/src/kernel.rs:1215-1435, 818-865).
// ---------------------------------------------------------------------------
namespace {

using Launcher = int (*)(ipus_context*, void*, const void* const*, const uint32_t*);
// Scalar constraints that validate_kernel_run enforces before any launch
// (kernel.rs:1384-1435): 0, or the status the run is rejected with.
using Checker = int (*)(const uint32_t*);

struct KernelEntry {
  const char* symbol;
  int inputs;
  std::vector<const char*> scalars;
  Launcher launch;
  Checker check = nullptr;
};

inline float bits_to_float(uint32_t bits) {
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// GemmArgs from the GEMM symbols' first eight scalars (batches, rows,
// columns, inner, transpose_left, transpose_right, left and right batch
// strides).
int gemm_args(void* out, const void* const* in, const uint32_t* s, GemmArgs* a) {
  if (s[4] > 1 || s[5] > 1) return IPUS_ERROR_INVALID_ARGUMENT;
  a->out = out;
  a->left = in[0];
  a->right = in[1];
  a->batches = s[0];
  a->rows = s[1];
  a->columns = s[2];
  a->inner = s[3];
  a->transpose_left = s[4] != 0;
  a->transpose_right = s[5] != 0;
  a->left_batch_stride = s[6];
  a->right_batch_stride = s[7];
  return 0;
}

int check_gemm_flags(const uint32_t* s) {
  return s[4] > 1 || s[5] > 1 ? IPUS_ERROR_INVALID_ARGUMENT : 0;
}

int run_gemm(ipus_context* ctx, void* out, const void* const* in, const uint32_t* s, bool f16,
             bool gelu = false) {
  GemmArgs a;
  if (int e = gemm_args(out, in, s, &a)) return e;
  a.gelu = gelu;
  return f16 ? launch_gemm_f16(ctx->stream, a) : launch_gemm_f32(ctx->stream, a);
}

// Attention launch from the registry scalars; `heads` (query, key, value) is
// null for the contiguous symbol.
int run_attention(ipus_context* c, void* o, const void* const* i, const uint32_t* s,
                  const uint32_t* heads) {
  AttentionArgs a;
  a.out = o;
  a.query = i[0];
  a.key = i[1];
  a.value = i[2];
  a.streams = s[0];
  a.query_rows = s[1];
  a.key_rows = s[2];
  a.width = s[3];
  a.value_width = s[4];
  a.scale = s[5] == 0 ? 1.0f / std::sqrt((float)s[3]) : bits_to_float(s[5]);
  a.causal = s[6] != 0;
  a.output_f16 = s[7] != 0;
  if (s[6] > 1 || s[7] > 1) return IPUS_ERROR_INVALID_ARGUMENT;
  if (heads)
    for (int k = 0; k < 3; ++k) a.heads[k] = heads[k];
  return launch_attention_f16(c->stream, a);
}

const std::vector<KernelEntry>& registry() {
  static const std::vector<KernelEntry> entries = {
      {"ipu_stack_gemm_f16", 2,
       {"batches", "rows", "columns", "inner", "transpose_left", "transpose_right",
        "left_batch_stride", "right_batch_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_gemm(c, o, i, s, true);
       }},
      // Gemm followed by Gelu of its fp16 result, fused into the GEMM
      // epilogue (no reference counterpart: build_package emits it for a
      // Gemm whose result only feeds one Gelu).
      {"ipu_stack_gemm_f16_gelu", 2,
       {"batches", "rows", "columns", "inner", "transpose_left", "transpose_right",
        "left_batch_stride", "right_batch_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_gemm(c, o, i, s, true, true);
       }},
      // C = addend + A . B (the reference's accumulate mode, gemm_f16_amp.S:
      // 43-52, 290-363, as one operator-level launch; also the residual
      // x + x . W that build_package fuses): the product rounded to fp16,
      // then added like ipu_stack_add_f16.  The addend may be the output.
      {"ipu_stack_gemm_f16_accumulate", 3,
       {"batches", "rows", "columns", "inner", "transpose_left", "transpose_right",
        "left_batch_stride", "right_batch_stride", "addend_batch_stride", "addend_row_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         GemmArgs a;
         if (int e = gemm_args(o, i, s, &a)) return e;
         a.addend = i[2];
         a.addend_batch_stride = s[8];
         a.addend_row_stride = s[9];
         return launch_gemm_f16(c->stream, a);
       },
       check_gemm_flags},
      // Split-K GEMM (no reference counterpart; planned by build_package for
      // few-tile, long-K shapes): fp32 partials float[splits][batches][M][N].
      {"ipu_stack_gemm_f16_split", 2,
       {"batches", "rows", "columns", "inner", "transpose_left", "transpose_right",
        "left_batch_stride", "right_batch_stride", "splits"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         if (s[4] > 1 || s[5] > 1) return IPUS_ERROR_INVALID_ARGUMENT;
         GemmArgs a;
         a.out = o;
         a.left = i[0];
         a.right = i[1];
         a.batches = s[0];
         a.rows = s[1];
         a.columns = s[2];
         a.inner = s[3];
         a.transpose_left = s[4] != 0;
         a.transpose_right = s[5] != 0;
         a.left_batch_stride = s[6];
         a.right_batch_stride = s[7];
         return launch_gemm_f16_split(c->stream, a, s[8]);
       }},
      // Sum of the split partials rounded to fp16 (GELU of it when gelu = 1).
      {"ipu_stack_reduce_splits_f16", 1, {"splits", "element_count", "gelu"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_reduce_splits_f16(c->stream, o, i[0], s[0], s[1], s[2] != 0);
       },
       [](const uint32_t* s) { return s[2] > 1 ? IPUS_ERROR_INVALID_ARGUMENT : 0; }},
      // The same sum plus an addend (the split form of
      // ipu_stack_gemm_f16_accumulate); partials [splits][batches][rows][columns].
      {"ipu_stack_reduce_splits_accumulate_f16", 2,
       {"splits", "batches", "rows", "columns", "addend_batch_stride", "addend_row_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         const SplitAddend add{i[1], s[2], s[3], s[4], s[5]};
         return launch_reduce_splits_f16(c->stream, o, i[0], s[0], (uint64_t)s[1] * s[2] * s[3],
                                         false, &add);
       }},
      {"ipu_stack_gemm_f32", 2,
       {"batches", "rows", "columns", "inner", "transpose_left", "transpose_right",
        "left_batch_stride", "right_batch_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_gemm(c, o, i, s, false);
       }},
      {"ipu_stack_flash_attention_online_f16", 3,
       {"matrices", "query_rows", "key_rows", "query_dimension", "value_dimension", "scale_bits",
        "causal", "output_f16"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_attention(c, o, i, s, nullptr);
       }},
      {"ipu_stack_flash_attention_heads_f16", 3,
       {"matrices", "query_rows", "key_rows", "query_dimension", "value_dimension", "scale_bits",
        "causal", "output_f16", "query_heads", "key_heads", "value_heads"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_attention(c, o, i, s, s + 8);
       }},
      {"ipu_stack_gelu_tanh_approx_f16", 1, {"element_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_gelu_f16(c->stream, o, i[0], s[0]);
       },
       // validate_kernel_run: the element count must be even (kernel.rs:1400-1413).
       [](const uint32_t* s) { return s[0] % 2 != 0 ? IPUS_ERROR_UNSUPPORTED_COUNT : 0; }},
      {"ipu_stack_reduce_sum_f16", 2, {"num_partials", "element_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_reduce_sum_f16(c->stream, o, i[0], i[1], s[0], s[1]);
       },
       // partials >= 2 (one initial + >= 1 remote) and count % 8 == 0
       // (kernel.rs:1414-1423).
       [](const uint32_t* s) {
         return s[0] < 1 || s[1] % 8 != 0 ? IPUS_ERROR_UNSUPPORTED_COUNT : 0;
       }},
      {"ipu_stack_rearrange_row_major_f16", 1,
       {"logical_rows", "physical_rows", "target_order", "logical_columns", "physical_columns",
        "row_block", "column_block", "matrices"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_rearrange_f16(c->stream, o, i[0], s[2], s[5], s[6], s[7], s[0], s[1], s[3],
                                     s[4]);
       }},
      {"ipu_stack_unpack_amp_f16", 1,
       {"matrices", "logical_rows", "physical_rows", "logical_columns", "physical_columns",
        "source_order"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_unpack_f16(c->stream, o, i[0], s[5], s[0], s[1], s[2], s[3], s[4]);
       }},
      {"ipu_stack_transpose_f16", 1, {"matrices", "rows", "columns"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_transpose_f16(c->stream, o, i[0], s[0], s[1], s[2]);
       }},
      {"ipu_stack_reduce_rows_f16", 1,
       {"rows", "columns", "source_order", "row_block", "column_block"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_reduce_rows_f16(c->stream, (float*)o, i[0], s[2], s[3], s[4], s[0], s[1]);
       }},
      {"ipu_stack_fill_zero", 0, {"byte_count"},
       [](ipus_context* c, void* o, const void* const*, const uint32_t* s) {
         return launch_fill_zero(c->stream, o, s[0]);
       }},
      // The reference's own FillZero step (emit.rs:38, kernel.rs:1223-1229):
      // bytes / 8 words dealt to six IPU workers, words_per_worker =
      // bytes / 8 / 6 and remainder_workers = bytes / 8 % 6 (kernel.rs:
      // 1174-1175), so the zeroed bytes are 8 (6 w + r).
      {"ipu_stack_fill_zero_u64", 0, {"words_per_worker", "remainder_workers"},
       [](ipus_context* c, void* o, const void* const*, const uint32_t* s) {
         return launch_fill_zero(c->stream, o, 8ull * (6ull * s[0] + s[1]));
       },
       [](const uint32_t* s) { return s[1] >= 6 ? IPUS_ERROR_INVALID_ARGUMENT : 0; }},
      {"ipu_stack_cast_f32_f16", 1, {"element_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_cast_f32_to_f16(c->stream, o, i[0], s[0]);
       }},
      {"ipu_stack_cast_f16_f32", 1, {"element_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_cast_f16_to_f32(c->stream, o, i[0], s[0]);
       }},
      {"ipu_stack_add_f16", 2, {"element_count", "left_broadcast_stride", "right_broadcast_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_flat_add(c, o, i, s, 1);
       }},
      {"ipu_stack_add_f32", 2, {"element_count", "left_broadcast_stride", "right_broadcast_stride"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_flat_add(c, o, i, s, 2);
       }},
      // Plan-internal symbols (no reference counterpart): general numpy
      // broadcasting add, split_heads copy, stored order -> row-major, GELU
      // of any element count, byte copy.
      {"ipu_stack_add_broadcast_f16", 2,
       {"rank", "shape0", "shape1", "shape2", "shape3", "shape4", "shape5", "left_stride0",
        "left_stride1", "left_stride2", "left_stride3", "left_stride4", "left_stride5",
        "right_stride0", "right_stride1", "right_stride2", "right_stride3", "right_stride4",
        "right_stride5"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_broadcast_add(c, o, i, s, 1);
       }},
      {"ipu_stack_add_broadcast_f32", 2,
       {"rank", "shape0", "shape1", "shape2", "shape3", "shape4", "shape5", "left_stride0",
        "left_stride1", "left_stride2", "left_stride3", "left_stride4", "left_stride5",
        "right_stride0", "right_stride1", "right_stride2", "right_stride3", "right_stride4",
        "right_stride5"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return run_broadcast_add(c, o, i, s, 2);
       }},
      {"ipu_stack_split_heads", 1, {"batch", "rows", "heads", "channels", "element_bytes"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_split_heads(c->stream, o, i[0], s[0], s[1], s[2], s[3], s[4]);
       }},
      {"ipu_stack_rearrange_to_row_major_f16", 1,
       {"source_order", "row_block", "column_block", "matrices", "rows", "columns"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_to_row_major_f16(c->stream, o, i[0], s[0], s[1], s[2], s[3], s[4], s[5]);
       }},
      // Declared input format -> row-major: input 0 the host bytes (the
      // shards in tile order), input 1 the shard table (tiling.h).
      {"ipu_stack_unshard", 2,
       {"shards", "rank", "order", "row_block", "column_block", "element_bytes",
        "max_shard_elements"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_unshard(c->stream, o, i[0], i[1], s[0], s[1], s[2], s[3], s[4], s[5],
                               s[6]);
       }},
      {"ipus_gelu_f16", 1, {"element_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_gelu_f16(c->stream, o, i[0], s[0]);
       }},
      // Roofline calibration (no reference counterpart): sustained MFMA rate
      // and shader clock for the given operand pattern.
      {"ipus_calibrate_mfma_f16", 1, {"operand_count", "iterations", "blocks"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_calibrate_mfma_f16(c->stream, o, i[0], s[0], s[1], s[2]);
       }},
      {"ipus_calibrate_mfma_f16_16x16x32", 1, {"operand_count", "iterations", "blocks"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_calibrate_mfma_f16(c->stream, o, i[0], s[0], s[1], s[2], true);
       }},
      {"ipus_calibrate_copy", 1, {"byte_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_calibrate_copy(c->stream, o, i[0], s[0]);
       }},
      {"ipu_stack_copy", 1, {"byte_count"},
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s) {
         return launch_copy(c->stream, o, i[0], s[0]);
       }},
  };
  return entries;
}

// ---- reference per-shape symbols ----
// The reference links one specialization per operand shape and names it by
// that shape (KernelBuildPlan::from_program: unpack kernel.rs:321-328,
// rearrange 374-379 with rearrangement_specialization 1122-1146, flash
// attention 506-515).  Here one generic kernel serves every shape, so such a
// symbol resolves to a launch of it whose shape comes from the suffix.
struct ShapeFamily {
  const char* prefix;
  // Suffix fields after the prefix: '#' a decimal u32, 'H' exactly eight
  // lowercase hex digits ({:08x}); any other character must match itself.
  const char* pattern;
  int inputs;
  std::vector<const char*> scalars;
  int (*check)(const uint32_t* shape, const uint32_t* scalars);
  int (*launch)(ipus_context*, void*, const void* const*, const uint32_t* scalars,
                const uint32_t* shape);
};

bool parse_suffix(const char* text, const char* pattern, uint32_t* fields) {
  int n = 0;
  for (; *pattern; ++pattern) {
    if (*pattern == '#') {
      if (*text < '0' || *text > '9') return false;
      uint64_t v = 0;
      int digits = 0;
      while (*text >= '0' && *text <= '9') {
        v = v * 10 + (uint64_t)(*text++ - '0');
        if (++digits > 10 || v > 0xffffffffull) return false;
      }
      fields[n++] = (uint32_t)v;
    } else if (*pattern == 'H') {
      uint32_t v = 0;
      for (int d = 0; d < 8; ++d, ++text) {
        const char ch = *text;
        if (ch >= '0' && ch <= '9') v = v * 16 + (uint32_t)(ch - '0');
        else if (ch >= 'a' && ch <= 'f') v = v * 16 + (uint32_t)(ch - 'a' + 10);
        else return false;
      }
      fields[n++] = v;
    } else if (*text++ != *pattern) {
      return false;
    }
  }
  return *text == '\0';
}

const std::vector<ShapeFamily>& shape_families() {
  static const std::vector<ShapeFamily> families = {
      // Row-major -> AMP-Left / AMP-TransposedRight / block-major, suffix
      // o{target}_r{logical rows}_p{physical rows}_c{logical columns}_p{physical
      // columns}; scalars as the reference passes them (kernel.rs:1351-1361).
      // A zero logical extent in the suffix is rearrangement_specialization's
      // runtime form (physical rows 64, fewer logical rows, kernel.rs:
      // 1129-1139; rearrange_f16.cpp reads the scalar when the define is 0).
      // The suffix does not name a block shape: target 2 is block-major
      // {row_block 64, column_block 16}, the only one the reference plans for
      // this conversion (layout.rs:356-361, 515-527).
      {"ipu_stack_rearrange_row_major_to_amp_f16_", "o#_r#_p#_c#_p#", 1,
       {"logical_rows", "physical_rows", "target_order", "logical_columns", "physical_columns"},
       [](const uint32_t* f, const uint32_t* s) {
         if (f[0] > 2 || s[2] != f[0]) return IPUS_ERROR_INVALID_ARGUMENT;
         if (s[1] != f[2] || s[4] != f[4]) return IPUS_ERROR_INVALID_ARGUMENT;
         if ((f[1] != 0 && s[0] != f[1]) || (f[3] != 0 && s[3] != f[3]))
           return IPUS_ERROR_INVALID_ARGUMENT;
         return 0;
       },
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s, const uint32_t* f) {
         return launch_rearrange_f16(c->stream, o, i[0], f[0], 64, 16, 1, s[0], s[1], s[3], s[4]);
       }},
      // AMP-Output / AMP-TransposedLeft -> row-major, suffix as above with the
      // source order (kernel.rs:321-328); the codelet compiles every extent in
      // and takes only `matrices` at run time (unpack_amp_f16.cpp:6-40), so
      // the scalar extents must equal the suffix.
      {"ipu_stack_unpack_amp_to_row_major_f16_", "o#_r#_p#_c#_p#", 1,
       {"matrices", "logical_rows", "physical_rows", "logical_columns", "physical_columns"},
       [](const uint32_t* f, const uint32_t* s) {
         if (f[0] > 1) return IPUS_ERROR_INVALID_ARGUMENT;
         for (int k = 1; k < 5; ++k)
           if (s[k] != f[k]) return IPUS_ERROR_INVALID_ARGUMENT;
         return 0;
       },
       [](ipus_context* c, void* o, const void* const* i, const uint32_t* s, const uint32_t* f) {
         return launch_unpack_f16(c->stream, o, i[0], f[0], s[0], s[1], s[2], s[3], s[4]);
       }},
      // Fused non-causal attention with fp32 output, suffix
      // m{matrices}_q{query rows}_k{key rows}_d{query width}_v{value width}_
      // {scale bits, {:08x}} (AttentionKernelShape, kernel.rs:121-129,
      // 986-1040); no scalars.
      {"ipu_stack_flash_attention_online_f16_", "m#_q#_k#_d#_v#_H", 3, {},
       [](const uint32_t*, const uint32_t*) { return 0; },
       [](ipus_context* c, void* o, const void* const* i, const uint32_t*, const uint32_t* f) {
         AttentionArgs a;
         a.out = o;
         a.query = i[0];
         a.key = i[1];
         a.value = i[2];
         a.streams = f[0];
         a.query_rows = f[1];
         a.key_rows = f[2];
         a.width = f[3];
         a.value_width = f[4];
         a.scale = bits_to_float(f[5]);
         a.causal = false;
         a.output_f16 = false;
         return launch_attention_f16(c->stream, a);
       }},
  };
  return families;
}

// Reference symbols this library does not forward, with the reason.
struct NotForwarded {
  const char* prefix;
  bool exact;  // the whole symbol, not a prefix
  int status;
  const char* reason;
};

const NotForwarded kNotForwarded[] = {
    {"ipu_stack_gemm_f16_init_", false, IPUS_ERROR_TRANSLATED,
     "a reference tile GEMM codelet (one AMP-Left x block-major shard, shape compiled in, "
     "kernel.rs:185-193) is translated per operator: one ipu_stack_gemm_f16 over the whole "
     "M, N, K"},
    {"ipu_stack_gemm_f16_accumulate_", false, IPUS_ERROR_TRANSLATED,
     "a reference tile GEMM codelet (accumulate mode) is translated per operator: one "
     "ipu_stack_gemm_f16_accumulate over the whole M, N, K"},
    {"ipu_stack_gemm_f32_init_", false, IPUS_ERROR_TRANSLATED,
     "a reference tile GEMM codelet is translated per operator: one ipu_stack_gemm_f32 over "
     "the whole M, N, K"},
    {"ipu_stack_gemm_f32_accumulate_", false, IPUS_ERROR_TRANSLATED,
     "a reference tile GEMM codelet (accumulate mode) is translated per operator: one "
     "ipu_stack_gemm_f32 plus ipu_stack_add_f32"},
    {"ipu_stack_attention_softmax_", false, IPUS_ERROR_TRANSLATED,
     "a staged-attention codelet (low.rs:2250-2463) is translated: the whole attention is one "
     "ipu_stack_flash_attention_online_f16 launch"},
    {"ipu_stack_attention_merge_", false, IPUS_ERROR_TRANSLATED,
     "a staged-attention codelet (low.rs:2250-2463) is translated: the whole attention is one "
     "ipu_stack_flash_attention_online_f16 launch"},
    {"ipu_stack_gemm_f8_", false, IPUS_ERROR_UNAVAILABLE,
     "fp8 GEMM is KernelAvailability::Required in the reference (kernel.rs:1544-1548): no "
     "device kernel there or here"},
    {"ipu_stack_cast_f8_", false, IPUS_ERROR_UNAVAILABLE, "fp8 casts have no device kernel"},
    {"ipu_stack_unsupported_", false, IPUS_ERROR_UNAVAILABLE,
     "the reference's placeholder for an unsupported kernel (kernel.rs:1252, 1516)"},
    {"ipu_stack_cast_identity", true, IPUS_ERROR_UNAVAILABLE,
     "a cast between equal precisions is KernelAvailability::Required in the reference "
     "(kernel.rs:1519-1529): no device kernel there or here"},
    {"ipu_stack_rearrange", true, IPUS_ERROR_UNAVAILABLE,
     "the reference's generic Rearrange is KernelAvailability::Required (kernel.rs:1365-1370): "
     "no device kernel there; ipu_stack_rearrange_row_major_f16 and "
     "ipu_stack_rearrange_to_row_major_f16 cover the row-major conversions"},
};

// One symbol resolved against the registry: a static entry, or a reference
// per-shape symbol with its shape fields.
struct Resolved {
  const KernelEntry* entry = nullptr;
  const ShapeFamily* family = nullptr;
  uint32_t shape[8] = {};
  int inputs() const { return entry ? entry->inputs : family->inputs; }
  const std::vector<const char*>& scalars() const {
    return entry ? entry->scalars : family->scalars;
  }
};

int resolve(const char* symbol, Resolved* r) {
  if (!symbol) return fail(IPUS_ERROR_UNKNOWN_SYMBOL, "kernel symbol is null");
  for (const auto& e : registry())
    if (strcmp(e.symbol, symbol) == 0) {
      r->entry = &e;
      return 0;
    }
  for (const auto& f : shape_families()) {
    const size_t n = strlen(f.prefix);
    if (strncmp(symbol, f.prefix, n) != 0) continue;
    if (!parse_suffix(symbol + n, f.pattern, r->shape))
      return fail(IPUS_ERROR_UNKNOWN_SYMBOL, "kernel symbol %s: suffix does not match %s%s",
                  symbol, f.prefix, f.pattern);
    r->family = &f;
    return 0;
  }
  if (strncmp(symbol, "ipu_stack_cast_", 15) == 0 && strstr(symbol, "_f8"))
    return fail(IPUS_ERROR_UNAVAILABLE, "kernel %s: fp8 casts have no device kernel", symbol);
  for (const auto& nf : kNotForwarded)
    if (nf.exact ? strcmp(symbol, nf.prefix) == 0
                 : strncmp(symbol, nf.prefix, strlen(nf.prefix)) == 0)
      return fail(nf.status, "kernel %s: %s", symbol, nf.reason);
  return fail(IPUS_ERROR_UNKNOWN_SYMBOL, "unknown kernel symbol %s", symbol);
}

// Interned copies of resolved per-shape symbols, so ipus_kernel_abi can hand
// out a pointer that stays valid until the process ends.
const char* intern(const char* symbol) {
  static std::mutex mutex;
  static std::set<std::string> names;
  std::lock_guard<std::mutex> lock(mutex);
  return names.insert(symbol).first->c_str();
}

void fill_info(const char* symbol, const Resolved& r, ipus_kernel_abi_info* info) {
  memset(info, 0, sizeof(*info));
  info->symbol = r.entry ? r.entry->symbol : intern(symbol);
  info->input_count = r.inputs();
  const auto& scalars = r.scalars();
  info->scalar_count = (int)scalars.size();
  for (size_t k = 0; k < scalars.size() && k < IPUS_MAX_SCALARS; ++k)
    info->scalar_names[k] = scalars[k];
  info->implemented = 1;
}

// validate_kernel_run (kernel.rs:1384-1435): the symbol resolves, pointer
// arity and scalar count match its ABI, and the scalars meet its constraints.
int validate_run(const char* symbol, int input_count, const uint32_t* scalars, int scalar_count,
                 Resolved* r) {
  if (int status = resolve(symbol, r)) return status;
  if (input_count != r->inputs())
    return fail(IPUS_ERROR_POINTER_ARITY, "kernel run has %d pointer operands, ABI requires %d",
                input_count, r->inputs());
  if (scalar_count != (int)r->scalars().size())
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "kernel %s takes %d scalars, got %d", symbol,
                (int)r->scalars().size(), scalar_count);
  if (scalar_count && !scalars) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null scalars");
  int status = 0;
  if (r->entry && r->entry->check) status = r->entry->check(scalars);
  if (r->family) status = r->family->check(r->shape, scalars);
  if (status == IPUS_ERROR_UNSUPPORTED_COUNT)
    return fail(status, "kernel %s does not support this element count", symbol);
  if (status) return fail(status, "kernel %s: scalars do not meet its ABI", symbol);
  return 0;
}

}  // namespace

namespace ipus {
// out[i] = left[i % L] + right[i % R] with L, R the broadcast strides (operand
// element counts; each must divide the element count).
int run_flat_add(ipus_context* c, void* o, const void* const* i, const uint32_t* s, int precision) {
  const uint32_t count = s[0], L = s[1], R = s[2];
  if (L == 0 || R == 0 || count % L != 0 || count % R != 0) return IPUS_ERROR_INVALID_ARGUMENT;
  AddArgs a;
  a.out = o;
  a.left = i[0];
  a.right = i[1];
  a.precision = precision;
  // Express as a 3-axis broadcast: [count / max, max / min, min] handled by
  // two views, each operand repeating with its own period.
  if (L == R) {
    a.rank = 2;
    a.shape[0] = count / L;
    a.shape[1] = L;
    a.left_strides[0] = 0;
    a.left_strides[1] = 1;
    a.right_strides[0] = 0;
    a.right_strides[1] = 1;
  } else {
    const uint32_t big = L > R ? L : R, small = L > R ? R : L;
    if (big % small != 0) return IPUS_ERROR_INVALID_ARGUMENT;
    a.rank = 3;
    a.shape[0] = count / big;
    a.shape[1] = big / small;
    a.shape[2] = small;
    const bool left_big = L > R;
    a.left_strides[0] = 0;
    a.left_strides[1] = left_big ? small : 0;
    a.left_strides[2] = 1;
    a.right_strides[0] = 0;
    a.right_strides[1] = left_big ? 0 : small;
    a.right_strides[2] = 1;
  }
  return launch_add(c->stream, a);
}

// Scalars: rank, shape[6], left strides[6], right strides[6] (elements).
int run_broadcast_add(ipus_context* c, void* o, const void* const* i, const uint32_t* s,
                      int precision) {
  AddArgs a;
  a.out = o;
  a.left = i[0];
  a.right = i[1];
  a.precision = precision;
  a.rank = (int)s[0];
  if (a.rank < 0 || a.rank > 6) return IPUS_ERROR_INVALID_ARGUMENT;
  for (int k = 0; k < 6; ++k) {
    a.shape[k] = s[1 + k];
    a.left_strides[k] = s[7 + k];
    a.right_strides[k] = s[13 + k];
  }
  return launch_add(c->stream, a);
}
}  // namespace ipus

extern "C" int ipus_kernel_count(int* count) {
  if (!count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "count is null");
  *count = (int)registry().size();
  return 0;
}

extern "C" int ipus_kernel_abi_at(int index, ipus_kernel_abi_info* info) {
  if (!info || index < 0 || index >= (int)registry().size())
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "kernel index %d out of range", index);
  Resolved r;
  r.entry = &registry()[(size_t)index];
  fill_info(r.entry->symbol, r, info);
  return 0;
}

extern "C" int ipus_kernel_abi(const char* symbol, ipus_kernel_abi_info* info) {
  if (!info) return fail(IPUS_ERROR_INVALID_ARGUMENT, "info is null");
  Resolved r;
  if (int status = resolve(symbol, &r)) return status;
  fill_info(symbol, r, info);
  return 0;
}

extern "C" int ipus_validate_kernel_run(const char* symbol, int input_count,
                                        const uint32_t* scalars, int scalar_count) {
  Resolved r;
  return validate_run(symbol, input_count, scalars, scalar_count, &r);
}

extern "C" int ipus_launch(ipus_context* ctx, const char* symbol, void* output,
                           const void* const* inputs, int input_count, const uint32_t* scalars,
                           int scalar_count) {
  if (!ctx) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null context");
  Resolved r;
  if (int status = validate_run(symbol, input_count, scalars, scalar_count, &r)) return status;
  if (!output) return fail(IPUS_ERROR_INVALID_ARGUMENT, "kernel %s: null output", symbol);
  for (int k = 0; k < input_count; ++k)
    if (!inputs || !inputs[k])
      return fail(IPUS_ERROR_INVALID_ARGUMENT, "kernel %s: null input %d", symbol, k);
  if (ctx->inject_status != 0) {
    if (ctx->inject_after == 0) {
      const int status = ctx->inject_status;
      ctx->inject_status = 0;
      return fail(status, "kernel %s: injected launch failure (%d)", symbol, status);
    }
    --ctx->inject_after;
  }
  if (int e = use_device(ctx)) return e;
  const int status = r.entry ? r.entry->launch(ctx, output, inputs, scalars)
                             : r.family->launch(ctx, output, inputs, scalars, r.shape);
  return check_launch(status, symbol);
}

extern "C" int ipus_gemm_f16_split_noalloc(ipus_context* ctx, void* output, const void* left,
                                           const void* right, uint32_t batches, uint32_t rows,
                                           uint32_t columns, uint32_t inner, int transpose_left,
                                           int transpose_right, uint64_t left_batch_stride,
                                           uint64_t right_batch_stride, uint32_t splits,
                                           int gelu) {
  if (!ctx || !output || !left || !right) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null argument");
  if (batches > 65535 || splits == 0 || splits > 64)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "batches must be <= 65535 and splits in 1..64");
  // batches x rows x columns can pass 2^64 bytes: an overflowing product
  // must not slip under the limit.
  uint64_t need = 0;
  const bool over = __builtin_mul_overflow((uint64_t)batches, (uint64_t)rows, &need) ||
                    __builtin_mul_overflow(need, (uint64_t)columns, &need) ||
                    __builtin_mul_overflow(need, (uint64_t)splits * sizeof(float), &need);
  if (over || need > IPUS_SPLIT_SCRATCH_BYTES)
    return fail(IPUS_ERROR_UNSUPPORTED_COUNT,
                "split-K partials need %llu bytes; the no-allocation scratch holds %llu",
                over ? ~0ull : (unsigned long long)need,
                (unsigned long long)IPUS_SPLIT_SCRATCH_BYTES);
  if (int e = use_device(ctx)) return e;
  GemmArgs a;
  a.out = output;
  a.left = left;
  a.right = right;
  a.batches = batches;
  a.rows = rows;
  a.columns = columns;
  a.inner = inner;
  a.transpose_left = transpose_left != 0;
  a.transpose_right = transpose_right != 0;
  a.left_batch_stride = left_batch_stride;
  a.right_batch_stride = right_batch_stride;
  a.gelu = gelu != 0;
  return check_launch(launch_gemm_f16_split_noalloc(ctx->stream, ctx->device, a, splits),
                      "ipus_gemm_f16_split_noalloc");
}

// ---------------------------------------------------------------------------
// Synthetic inputs
// ---------------------------------------------------------------------------
namespace {

inline uint64_t splitmix64(uint64_t state) {
  uint64_t z = state + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

inline float synth_value(uint64_t seed, uint32_t tensor, uint64_t i, int dist, float scale) {
  const uint64_t z = splitmix64(seed ^ ((uint64_t)tensor << 48) ^ i);
  if (dist == 0) {
    // top 24 bits -> [-1, 1)
    const double u = (double)(z >> 40) * (1.0 / 16777216.0);
    return (float)(2.0 * u - 1.0) * scale;
  }
  // Box-Muller with u1 in (0, 1] from the high 32 bits, u2 from the low 32.
  const double u1 = ((double)(z >> 32) + 1.0) * (1.0 / 4294967296.0);
  const double u2 = (double)(z & 0xffffffffu) * (1.0 / 4294967296.0);
  const double r = std::sqrt(-2.0 * std::log(u1));
  return (float)(r * std::cos(6.283185307179586 * u2)) * scale;
}

uint16_t f32_to_f16_rne(float value) {
  uint32_t x;
  memcpy(&x, &value, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exponent = (x >> 23) & 0xffu;
  uint32_t mantissa = x & 0x7fffffu;
  if (exponent == 0xffu) return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x200u : 0u));
  const int32_t e = (int32_t)exponent - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mantissa |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    uint32_t r = mantissa >> shift;
    const uint32_t rem = mantissa & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((uint32_t)e << 10) | (mantissa >> 13);
  const uint32_t rem = mantissa & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

template <typename F>
void parallel_chunks(uint64_t count, F&& f) {
  unsigned threads = std::thread::hardware_concurrency();
  if (threads == 0) threads = 1;
  if (threads > 16) threads = 16;
  if (count < (1u << 16)) threads = 1;
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < threads; ++t)
    pool.emplace_back([&, t] { f(count * t / threads, count * (t + 1) / threads); });
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" int ipus_synth_f16(uint16_t* out, uint64_t count, uint64_t seed, uint32_t tensor,
                              int distribution, float scale) {
  if (!out && count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null output");
  if (distribution != 0 && distribution != 1)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "distribution must be 0 (uniform) or 1 (normal)");
  parallel_chunks(count, [&](uint64_t b, uint64_t e) {
    for (uint64_t i = b; i < e; ++i)
      out[i] = f32_to_f16_rne(synth_value(seed, tensor, i, distribution, scale));
  });
  return 0;
}

extern "C" int ipus_synth_f32(float* out, uint64_t count, uint64_t seed, uint32_t tensor,
                              int distribution, float scale) {
  if (!out && count) return fail(IPUS_ERROR_INVALID_ARGUMENT, "null output");
  if (distribution != 0 && distribution != 1)
    return fail(IPUS_ERROR_INVALID_ARGUMENT, "distribution must be 0 (uniform) or 1 (normal)");
  parallel_chunks(count, [&](uint64_t b, uint64_t e) {
    for (uint64_t i = b; i < e; ++i) out[i] = synth_value(seed, tensor, i, distribution, scale);
  });
  return 0;
}
