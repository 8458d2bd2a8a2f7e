// Internal host-side declarations shared by the libipus translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/ipus.h"

struct ipus_context {
  int device = 0;
  hipStream_t stream = nullptr;
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
