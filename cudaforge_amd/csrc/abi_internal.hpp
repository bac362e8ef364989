// abi_internal.hpp -- error reporting, device queries and the launch helper
// shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/cudaforge_amd.h"
#include "common.hpp"

namespace cfa {
namespace abi {

void clear_error();
int fail_arg(const char *msg);
int fail_hip(hipError_t e, const char *where);
int fail_code(int code, const char *msg);
int device_cu_count();

}  // namespace abi

namespace prof {
bool enabled();
void *begin(const char *name, hipStream_t stream);
void end(void *token, hipStream_t stream);
}  // namespace prof

}  // namespace cfa

// Launch `kernel` on `stream`, bracketed by profiling events when enabled;
// returns CFA_ERR_HIP from the enclosing function on a launch error.
#define CFA_LAUNCH(name, kernel, grid, block, shmem, stream, ...)                      \
  do {                                                                                 \
    void *cfa_prof_tok_ = ::cfa::prof::enabled() ? ::cfa::prof::begin(name, stream)    \
                                                 : nullptr;                            \
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);               \
    if (cfa_prof_tok_) ::cfa::prof::end(cfa_prof_tok_, stream);                        \
    if (hipError_t cfa_e_ = hipGetLastError()) return ::cfa::abi::fail_hip(cfa_e_, name); \
  } while (0)
