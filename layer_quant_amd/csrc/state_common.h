// Device helpers shared by the recurrent-state kernels (MX8/MX4 state in mx_state.hip, the
// plain bf16/fp16/fp32 state in ssm_state.hip): lane geometry, strided float loads, buffer
// descriptors and the state cache policy.
#pragma once

#include "lq_common.h"

namespace lq {

// Grid (ceil(P * vbpr / 256), H, B): one lane per 16-value block of one (b, h) pair; the N/16
// block lanes of a state row are adjacent (vbpr = N/16 rounded up to a power of two). Batch and
// head come from the block index, so every per-(b, h) offset is uniform and lane offsets are
// 32-bit.
struct LaneIdx {
  int b, h, pp, blk;
  bool in_range, active;
};

__device__ __forceinline__ LaneIdx lane_index(int P, int vbpr_log2, int bpr) {
  LaneIdx L;
  L.h = blockIdx.y;
  L.b = blockIdx.z;
  const int lanes = P << vbpr_log2;
  int idx = blockIdx.x * 256 + threadIdx.x;
  L.in_range = idx < lanes;
  if (!L.in_range) idx = lanes - 1;  // whole trailing row groups only; they store nothing
  L.pp = idx >> vbpr_log2;
  const int blk = idx & ((1 << vbpr_log2) - 1);
  L.active = L.in_range && blk < bpr;
  L.blk = min(blk, bpr - 1);
  return L;
}

__device__ __forceinline__ int dtype_bytes(int dtype) {
  return dtype == LQ_F32 ? 4 : 2;
}

// uniform base of a strided float view at (i0, i1) of its leading dimensions
__device__ __forceinline__ const char* vbase(const View& v, int i0, int i1) {
  return (const char*)v.data + ((int64_t)i0 * v.s[0] + (int64_t)i1 * v.s[1]) * dtype_bytes(v.dtype);
}

__device__ __forceinline__ float ldf(const char* base, int dtype, int idx) {
  switch (dtype) {
    case LQ_BF16:
      return bf16_bits_to_float(((const uint16_t*)base)[idx]);
    case LQ_F16:
      return (float)(((const _Float16*)base)[idx]);
    default:
      return ((const float*)base)[idx];
  }
}


// 16 consecutive d_state values of B or C: vector loads for contiguous bf16 (BCVEC), else
// strided element loads of any float dtype.
template <bool BCVEC>
__device__ __forceinline__ void load16(const char* base, int dtype, int stride, int n0,
                                       float (&o)[16]) {
  if constexpr (BCVEC) {
    const uint4* p4 = (const uint4*)((const uint16_t*)base + n0);
    const uint4 a = p4[0];
    const uint4 b = p4[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = ldf(base, dtype, (n0 + i) * stride);
  }
}


typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int BUF_DWORD3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)
// Cache policy bits of the recurrent state's buffer loads and stores (gfx950 CPol: sc0 = 1,
// nt = 2, sc1 = 16). Every state byte is read once and written once per update, and one update of
// a Nemotron-H layer at batch 64 (212 MB in MX4) would only evict other data from L2 and the
// Infinity Cache: loads stream (nt), stores stream through to memory (nt | sc1). Measured on the
// MX4 update at batch 64: 51 us with the default policy, 48.6 us with nt loads only, 44.3-45.4 us
// with streaming stores as well.
constexpr int STATE_LOAD_POLICY = 2;
constexpr int STATE_STORE_POLICY = 18;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, BUF_DWORD3);
}

// Element at a wave-uniform address, read by a scalar load of the aligned 32-bit word holding it
// (a 4-byte aligned word never crosses a page, so it stays inside the allocation's pages).
__device__ __forceinline__ uint32_t uniform_word(const char* addr) {
  typedef const __attribute__((address_space(4))) uint32_t* cword_t;
  return *(cword_t)((uintptr_t)addr & ~(uintptr_t)3);
}

__device__ __forceinline__ float uniform_elem(const char* addr, int dtype) {
  return word_elem(uniform_word(addr), (uint32_t)((uintptr_t)addr & 2u) * 8u, dtype);
}

// Row-sum over the 2^BPR_LOG2 adjacent lanes of a state row with DPP moves: quad swaps, then the
// half-row mirror (lane i <-> 7 - i) and the row mirror (i <-> 15 - i), each pairing every lane
// with one in the other half of its group.
template <int BPR_LOG2>
__device__ __forceinline__ float row_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
  if constexpr (BPR_LOG2 >= 3) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
  }
  if constexpr (BPR_LOG2 >= 4) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
  }
  return v;
}


// 16 bf16 values of B or C for the lane's block column (two 16-byte loads).
template <class Params>
__device__ __forceinline__ void load_bc(const Params& p, int b, int grp, uint32_t n0,
                                        uint32_t N, u32x4_t (&bw)[2], u32x4_t (&cw)[2]) {
  const auto rB = make_buf(vbase(p.B, b, grp), N * 2);
  const auto rC = make_buf(vbase(p.C, b, grp), N * 2);
  bw[0] = __builtin_amdgcn_raw_buffer_load_b128(rB, n0 * 2, 0, 0);
  bw[1] = __builtin_amdgcn_raw_buffer_load_b128(rB, n0 * 2 + 16, 0, 0);
  cw[0] = __builtin_amdgcn_raw_buffer_load_b128(rC, n0 * 2, 0, 0);
  cw[1] = __builtin_amdgcn_raw_buffer_load_b128(rC, n0 * 2 + 16, 0, 0);
}

__device__ __forceinline__ void expand_bf16(const u32x4_t (&w)[2], float (&o)[16]) {
  const uint32_t a[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[2 * i] = __uint_as_float(a[i] << 16);
    o[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
  }
}

// Head scalars (hybrid_quant/mamba_state_8b_kernel.py:134-139): dt (+ dt_bias, softplus), exp(A dt) and D of head h. Without
// dt_bias or D the host points their views at dt with zero strides, so every scalar load is
// unconditional. exp and log use the hardware transcendentals (relative error ~1e-6, far inside
// the 2e-3 output tolerance).
struct HeadScalars {
  float dt, dA, D;
};

template <class Params>
__device__ __forceinline__ HeadScalars head_scalars(const Params& p, int b, int h) {
  HeadScalars s;
  // all four words are loaded before any dtype conversion (a branch), so that the loads go out
  // together instead of one memory round trip after another
  const char* a_dt = vbase(p.dt, b, h);
  const char* a_dtb = vbase(p.dtb, h, 0);
  const char* a_A = vbase(p.A, h, 0);
  const char* a_D = vbase(p.D, h, 0);
  uint32_t w_dt = uniform_word(a_dt), w_dtb = uniform_word(a_dtb);
  uint32_t w_A = uniform_word(a_A), w_D = uniform_word(a_D);
  asm volatile("" : "+s"(w_dt), "+s"(w_dtb), "+s"(w_A), "+s"(w_D));  // one wait for all four
  auto sh = [](const char* a) { return (uint32_t)((uintptr_t)a & 2u) * 8u; };
  float dtv = word_elem(w_dt, sh(a_dt), p.dt.dtype);
  const float dtb = word_elem(w_dtb, sh(a_dtb), p.dtb.dtype);
  const float av = word_elem(w_A, sh(a_A), p.A.dtype);
  s.D = word_elem(w_D, sh(a_D), p.D.dtype);
  if (p.has_dtb) dtv += dtb;
  if (p.softplus) dtv = dtv <= 20.0f ? __logf(1.0f + __expf(dtv)) : dtv;
  s.dt = dtv;
  s.dA = __expf(av * dtv);
  return s;
}

}  // namespace lq
