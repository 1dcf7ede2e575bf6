// Host side of the C ABI shared by every entry point: version, thread-local error message,
// descriptor validation.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>

#include "lq_common.h"

namespace lq {

static thread_local std::string g_last_error;

static void vset_error(const char* fmt, va_list ap) {
  char buf[1024];
  vsnprintf(buf, sizeof(buf), fmt, ap);
  g_last_error = buf;
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset_error(fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset_error(fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(LQ_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return LQ_OK;
}

int check_tensor(const lq_tensor* t, const char* name, int ndim, bool float_dtype,
                 int exact_dtype) {
  if (t == nullptr) return fail(LQ_ERR_INVALID_ARG, "%s: descriptor is NULL", name);
  if (t->data == nullptr) return fail(LQ_ERR_INVALID_ARG, "%s: data pointer is NULL", name);
  if (t->ndim != ndim) {
    return fail(LQ_ERR_INVALID_ARG, "%s: expected %d dims, got %d", name, ndim, t->ndim);
  }
  for (int i = 0; i < ndim; ++i) {
    if (t->shape[i] < 0) return fail(LQ_ERR_INVALID_ARG, "%s: negative extent", name);
  }
  if (exact_dtype >= 0 && t->dtype != exact_dtype) {
    return fail(LQ_ERR_INVALID_ARG, "%s: dtype code %d, expected %d", name, t->dtype,
                exact_dtype);
  }
  if (float_dtype && !is_float_dtype(t->dtype)) {
    return fail(LQ_ERR_INVALID_ARG, "%s: dtype code %d is not f32/f16/bf16", name, t->dtype);
  }
  if (dtype_size(t->dtype) == 0) {
    return fail(LQ_ERR_INVALID_ARG, "%s: unknown dtype code %d", name, t->dtype);
  }
  return LQ_OK;
}

// Environment names of the LQ_DIAG_* bits, in bit order.
static const char* const kDiagEnv[] = {
    "LQ_ATTN_FORCE_GENERIC", "LQ_ATTN_REQUIRE_FAST", "LQ_PREFILL_FORCE_GENERIC",
    "LQ_PREFILL_REQUIRE_MFMA", "LQ_MX_FORCE_GENERIC", "LQ_MX_REQUIRE_ROWS",
    "LQ_SSM_FORCE_GENERIC", "LQ_SSM_REQUIRE_ROWS", "LQ_ATTN_FOLD_MERGE"};

static uint32_t diag_from_env() {
  uint32_t flags = 0;
  for (uint32_t i = 0; i < sizeof(kDiagEnv) / sizeof(kDiagEnv[0]); ++i) {
    const char* v = getenv(kDiagEnv[i]);
    if (v != nullptr && v[0] != '\0' && v[0] != '0') flags |= 1u << i;
  }
  return flags;
}

// initialised while the library loads (before any entry point can run)
static std::atomic<uint32_t> g_diag{diag_from_env()};

bool diag(uint32_t bit) { return (g_diag.load(std::memory_order_relaxed) & bit) != 0; }

int64_t max_offset(const lq_tensor* t) {
  int64_t off = 0;
  for (int i = 0; i < t->ndim; ++i) {
    if (t->shape[i] == 0) return -1;
    off += (t->shape[i] - 1) * (t->stride[i] < 0 ? 0 : t->stride[i]);
  }
  return off;
}

}  // namespace lq

extern "C" int lq_abi_version(void) { return LQ_ABI_VERSION; }

extern "C" const char* lq_last_error(void) { return lq::g_last_error.c_str(); }

extern "C" uint32_t lq_diagnostics(void) { return lq::g_diag.load(std::memory_order_relaxed); }

extern "C" uint32_t lq_set_diagnostics(uint32_t flags) {
  return lq::g_diag.exchange(flags & LQ_DIAG_ALL, std::memory_order_relaxed);
}
