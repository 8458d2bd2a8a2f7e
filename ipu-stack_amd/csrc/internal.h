// Internal host-side declarations shared by the libipus translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/ipus.h"

#include <mutex>
#include <unordered_map>

struct ipus_context {
  int device = 0;
  hipStream_t stream = nullptr;
  // Buffers allocated through this context and not yet freed (pointer ->
  // bytes); ipus_context_destroy releases whatever is left.
  std::mutex live_mutex;
  std::unordered_map<void*, size_t> live;
  // Failure injection (ipus_context_inject_launch_failure): after
  // inject_after more launches, the next one returns inject_status.
  uint32_t inject_after = 0;
  int inject_status = 0;
};

namespace ipus {

// Records a formatted message as the thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
// Makes the context's device current for the calling thread.
int use_device(const ipus_context* ctx);
// Turns a launcher status into a recorded error for `symbol`.
int check_launch(int status, const char* symbol);

int run_flat_add(ipus_context* c, void* o, const void* const* i, const uint32_t* s, int precision);
int run_broadcast_add(ipus_context* c, void* o, const void* const* i, const uint32_t* s,
                      int precision);

}  // namespace ipus
