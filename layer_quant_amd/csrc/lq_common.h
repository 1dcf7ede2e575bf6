// Shared host and device helpers of liblayer_quant.so (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/layer_quant.h"

namespace lq {

// ---------------------------------------------------------------------------------------------
// host: error reporting and argument validation (no HIP call happens before validation passes)
// ---------------------------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

inline int dtype_size(int dtype) {
  switch (dtype) {
    case LQ_U8:
    case LQ_I8:
      return 1;
    case LQ_F16:
    case LQ_BF16:
      return 2;
    case LQ_F32:
    case LQ_I32:
      return 4;
    case LQ_I64:
      return 8;
    default:
      return 0;
  }
}

inline bool is_float_dtype(int dtype) {
  return dtype == LQ_F32 || dtype == LQ_F16 || dtype == LQ_BF16;
}

// Diagnostic switches (LQ_DIAG_* bits): taken from the environment once, when the library is
// loaded, and changed afterwards only by lq_set_diagnostics. Entry points read them with one
// relaxed atomic load, so no launch path calls getenv.
bool diag(uint32_t bit);

// Validates pointer, rank and dtype of a descriptor; returns 0 or an LQ_ERR code (message set).
int check_tensor(const lq_tensor* t, const char* name, int ndim, bool float_dtype,
                 int exact_dtype = -1);

// Largest element offset reachable through a descriptor (for bounds reasoning on the host).
int64_t max_offset(const lq_tensor* t);

// ---------------------------------------------------------------------------------------------
// device: dtype conversion
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (NaN -> canonical quiet NaN), as torch converts.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Float value of the 16- or 32-bit element held in the 32-bit word w at bit `shift` (0 or 16).
__device__ __forceinline__ float word_elem(uint32_t w, uint32_t shift, int dtype) {
  const uint32_t h16 = (w >> shift) & 0xffffu;
  if (dtype == LQ_F32) return __uint_as_float(w);
  if (dtype == LQ_BF16) return __uint_as_float(h16 << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// The aligned 32-bit word holding element idx of a bf16, fp16 or fp32 tensor, and the element's
// bit offset in it (for word_elem). A 4-byte aligned word never crosses a page, so the read stays
// inside the allocation's pages. Several such loads go out together and are converted after the
// last; load_float's dtype branch waits after each load.
__device__ __forceinline__ uint32_t elem_word(const void* base, int dtype, int64_t idx,
                                              uint32_t& shift) {
  const uintptr_t a = (uintptr_t)base + (uintptr_t)(idx * (dtype == LQ_F32 ? 4 : 2));
  shift = (uint32_t)(a & 2u) * 8u;
  typedef const __attribute__((address_space(1))) uint32_t* gword_t;  // a global load, not flat
  return *(gword_t)(a & ~(uintptr_t)3);
}

__device__ __forceinline__ float load_float(const void* base, int dtype, int64_t idx) {
  switch (dtype) {
    case LQ_BF16:
      return bf16_bits_to_float(((const uint16_t*)base)[idx]);
    case LQ_F16:
      return (float)(((const _Float16*)base)[idx]);
    default:
      return ((const float*)base)[idx];
  }
}

__device__ __forceinline__ void store_float(void* base, int dtype, int64_t idx, float v) {
  switch (dtype) {
    case LQ_BF16:
      ((uint16_t*)base)[idx] = float_to_bf16_bits(v);
      break;
    case LQ_F16:
      ((_Float16*)base)[idx] = (_Float16)v;
      break;
    default:
      ((float*)base)[idx] = v;
      break;
  }
}

// A strided view passed by value to kernels: base pointer, dtype code, up to 4 strides.
struct View {
  void* data;
  int dtype;
  int64_t s[4];
};

inline View make_view(const lq_tensor* t) {
  View v{};
  if (t == nullptr) return v;
  v.data = t->data;
  v.dtype = t->dtype;
  for (int i = 0; i < 4; ++i) v.s[i] = i < t->ndim ? t->stride[i] : 0;
  return v;
}

// ---------------------------------------------------------------------------------------------
// device: wave64 reductions
// ---------------------------------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace lq
