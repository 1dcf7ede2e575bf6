// INT4 group quantisation of one K or V token row, shared by the pack kernel and the decode
// attention's fused pack so that both write the same bytes.
#pragma once

#include "lq_common.h"

namespace lq {

// Lane j's byte of a token row (dims 2j and 2j + 1) and its group's scale, the group being the
// GH = g/2 adjacent lanes (a power of two <= 64, so a group never straddles a wave): absmax by a
// shuffle reduction, scale = max(absmax / 7, 1e-8), q = clamp(rint(x / scale), -8, 7) (IEEE
// division, round half to even), two's-complement nibbles with the even dim in the low nibble
// (reference hybrid_quant/int4_8b_attention.py:56-111). Every lane of the wave must be active.
template <int GH>
__device__ __forceinline__ uint32_t int4_quantize_pair(float v0, float v1, float& scale) {
  float amax = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
  for (int o = GH >> 1; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  scale = fmaxf(amax / 7.0f, 1.0e-8f);
  const int q0 = min(max((int)rintf(v0 / scale), -8), 7);
  const int q1 = min(max((int)rintf(v1 / scale), -8), 7);
  return (uint32_t)(((q1 & 15) << 4) | (q0 & 15));
}

// Validates the token tensors k, v [B, Hkv, T, D] (any float dtype and strides) against the
// packed caches and scales as lq_int4_pack_kv_pair does, for rows row .. row + T - 1 given on the
// host; with `launch`, packs them there (one launch for K and V) on `stream`.
int pack_pair_at(const lq_tensor* k, const lq_tensor* v, const lq_tensor* k_packed,
                 const lq_tensor* v_packed, const lq_tensor* k_scale, const lq_tensor* v_scale,
                 int64_t row, int group_size, bool launch, hipStream_t stream, const char* what);

}  // namespace lq
