// abi.cpp -- thread-local error state, device queries, version and the host
// uniform stream of the compatibility engine.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>
#include <random>
#include <string>

#include "abi_internal.hpp"

namespace cfa {
namespace abi {

static thread_local std::string g_last_error;

void clear_error() { g_last_error.clear(); }

int fail_arg(const char *msg) {
  g_last_error = msg;
  return CFA_ERR_ARG;
}

int fail_code(int code, const char *msg) {
  g_last_error = msg;
  return code;
}

int fail_hip(hipError_t e, const char *where) {
  g_last_error = std::string(where) + ": " + hipGetErrorString(e);
  return CFA_ERR_HIP;
}

// Compute-unit count of the current device, cached per device ordinal.
int device_cu_count() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace abi
}  // namespace cfa

extern "C" const char *cfa_last_error(void) { return cfa::abi::g_last_error.c_str(); }

extern "C" int cfa_version(void) { return CFA_ABI_VERSION; }

// ---------------------------------------------------------------------------
// Host uniform stream (speculative.cpp:8-9, 13-14, 64, 72).
// ---------------------------------------------------------------------------
struct cfa_rng {
  std::mt19937 engine;
};

extern "C" cfa_rng *cfa_rng_create(uint64_t seed) {
  cfa::abi::clear_error();
  // speculative.cpp:9 constructs rng_(config.rng_seed): mt19937's constructor
  // takes result_type, so the seed is reduced modulo 2^32.
  return new (std::nothrow) cfa_rng{std::mt19937(static_cast<std::mt19937::result_type>(seed))};
}

extern "C" void cfa_rng_destroy(cfa_rng *rng) { delete rng; }

extern "C" int cfa_rng_peek(const cfa_rng *rng, int n, float *out) {
  cfa::abi::clear_error();
  if (!rng || n < 0 || (n > 0 && !out)) return cfa::abi::fail_arg("cfa_rng_peek: bad arguments");
  std::mt19937 copy = rng->engine;
  std::uniform_real_distribution<float> dist(0.0f, 1.0f);
  for (int i = 0; i < n; ++i) out[i] = dist(copy);
  return CFA_OK;
}

extern "C" int cfa_rng_advance(cfa_rng *rng, int n) {
  cfa::abi::clear_error();
  if (!rng || n < 0) return cfa::abi::fail_arg("cfa_rng_advance: bad arguments");
  std::uniform_real_distribution<float> dist(0.0f, 1.0f);
  for (int i = 0; i < n; ++i) (void)dist(rng->engine);
  return CFA_OK;
}
