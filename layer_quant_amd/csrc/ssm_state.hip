// Plain (unquantized) Mamba2 selective-state update: one decode step of a bf16, fp16 or fp32
// recurrent state, in place.
//
// Replaces mamba-ssm 2.3.2.post1's selective_state_update, which the reference calls for every
// layer whose state is not registered for the MX kernel (hybrid_quant/mamba_state_8b_kernel.py:
// 738-747) and which is its bf16-state baseline. Semantics (fp32 arithmetic, state rounded back to
// its dtype with round-to-nearest-even):
//   dt' = softplus(dt + dt_bias)        (softplus only with dt_softplus; identity above 20)
//   h'  = h * exp(A dt') + (B dt') x    (one fma per element)
//   y   = sum_n h'_n C_n + D x,  y *= z * sigmoid(z) when z is given
// Geometry as the MX general kernel: one lane per 16-value block of a state row, the N/16 block
// lanes of a row adjacent, grid (ceil(P * vbpr / 256), H, B).
#include <math.h>
#include <stdlib.h>

#include "lq_common.h"
#include "state_common.h"

namespace lq {

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

struct SsmParams {
  View st, x, dt, dtb, A, B, C, D, z, out;
  int Bn, H, P, N, ratio, bpr, vbpr_log2;
  int has_dtb, has_D, has_z, softplus, a_row_const;
  uint32_t st_span;  // bytes of one (batch, head) state slice, for the vector path's descriptor
  // rows kernel: byte stride between rows of x, z and out, and the byte span of one
  // (batch, head) slice of each rounded up to 4 (0 for an absent z)
  uint32_t x_row_bytes, z_row_bytes, out_row_bytes;
  uint32_t x_span, z_span, out_span;
};

// 16 state values of one lane: buffer loads for a contiguous 16-byte aligned last dimension
// (VEC), element loads otherwise.
template <int SDT, bool VEC>
__device__ __forceinline__ void load_state16(const SsmParams& p, const char* sb, int pp, int n0,
                                             float (&h)[16]) {
  if constexpr (VEC) {
    const auto rs = make_buf(sb, p.st_span);
    constexpr int ES = SDT == LQ_F32 ? 4 : 2;
    const uint32_t off = (uint32_t)(pp * (int)p.st.s[2] + n0) * ES;
    if constexpr (SDT == LQ_F32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * j, 0, STATE_LOAD_POLICY);
        h[4 * j] = __uint_as_float(w.x);
        h[4 * j + 1] = __uint_as_float(w.y);
        h[4 * j + 2] = __uint_as_float(w.z);
        h[4 * j + 3] = __uint_as_float(w.w);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * j, 0, STATE_LOAD_POLICY);
        const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          h[8 * j + 2 * i] = word_elem(a[i], 0, SDT);
          h[8 * j + 2 * i + 1] = word_elem(a[i], 16, SDT);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) h[i] = ldf(sb, SDT, pp * (int)p.st.s[2] + (n0 + i) * (int)p.st.s[3]);
  }
}

template <int SDT>
__device__ __forceinline__ uint32_t to_bits16(float v) {
  if constexpr (SDT == LQ_BF16) {
    return float_to_bf16_bits(v);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

template <int SDT, bool VEC>
__device__ __forceinline__ void store_state16(const SsmParams& p, char* sb, int pp, int n0,
                                              const float (&h)[16]) {
  if constexpr (VEC) {
    const auto rs = make_buf(sb, p.st_span);
    constexpr int ES = SDT == LQ_F32 ? 4 : 2;
    const uint32_t off = (uint32_t)(pp * (int)p.st.s[2] + n0) * ES;
    if constexpr (SDT == LQ_F32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t w{__float_as_uint(h[4 * j]), __float_as_uint(h[4 * j + 1]),
                        __float_as_uint(h[4 * j + 2]), __float_as_uint(h[4 * j + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(w, rs, off + 16 * j, 0, STATE_STORE_POLICY);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint32_t a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = to_bits16<SDT>(h[8 * j + 2 * i]) | (to_bits16<SDT>(h[8 * j + 2 * i + 1]) << 16);
        }
        __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{a[0], a[1], a[2], a[3]}, rs, off + 16 * j, 0,
                                               STATE_STORE_POLICY);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      store_float(sb, SDT, pp * p.st.s[2] + (int64_t)(n0 + i) * p.st.s[3], h[i]);
    }
  }
}

template <int SDT, bool VEC, bool BCVEC>
__global__ __launch_bounds__(256) void ssm_update_kernel(SsmParams p) {
  const LaneIdx L = lane_index(p.P, p.vbpr_log2, p.bpr);
  const int b = L.b, h = L.h, pp = L.pp;
  const int n0 = L.blk * 16;
  char* sb = (char*)vbase(p.st, b, h);
  float hv[16];
  load_state16<SDT, VEC>(p, sb, pp, n0, hv);

  const float xv = ldf(vbase(p.x, b, h), p.x.dtype, pp * (int)p.x.s[2]);
  float dtv = ldf(vbase(p.dt, b, h), p.dt.dtype, pp * (int)p.dt.s[2]);
  if (p.has_dtb) dtv += ldf(vbase(p.dtb, h, 0), p.dtb.dtype, pp * (int)p.dtb.s[1]);
  if (p.softplus) dtv = dtv <= 20.0f ? __logf(1.0f + __expf(dtv)) : dtv;
  const int grp = h / p.ratio;
  float Bv[16], Cv[16];
  load16<BCVEC>(vbase(p.B, b, grp), p.B.dtype, (int)p.B.s[2], n0, Bv);
  load16<BCVEC>(vbase(p.C, b, grp), p.C.dtype, (int)p.C.s[2], n0, Cv);
  const char* ab = vbase(p.A, h, 0);
  const int aoff = pp * (int)p.A.s[1] + n0 * (int)p.A.s[2];

  float ypart = 0.0f;
  if (p.a_row_const) {
    const float dA = __expf(ldf(ab, p.A.dtype, aoff) * dtv);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      hv[i] = fmaf(hv[i], dA, (Bv[i] * dtv) * xv);
      ypart = fmaf(hv[i], Cv[i], ypart);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float dA = __expf(ldf(ab, p.A.dtype, aoff + i * (int)p.A.s[2]) * dtv);
      hv[i] = fmaf(hv[i], dA, (Bv[i] * dtv) * xv);
      ypart = fmaf(hv[i], Cv[i], ypart);
    }
  }
  if (!L.active) ypart = 0.0f;
  for (int o = (1 << p.vbpr_log2) >> 1; o > 0; o >>= 1) ypart += __shfl_xor(ypart, o, 64);
  if (L.in_range && L.blk == 0 && (threadIdx.x & ((1 << p.vbpr_log2) - 1)) == 0) {
    float y = ypart;
    if (p.has_D) y += xv * ldf(vbase(p.D, h, 0), p.D.dtype, pp * (int)p.D.s[1]);
    if (p.has_z) {
      const float zv = ldf(vbase(p.z, b, h), p.z.dtype, pp * (int)p.z.s[2]);
      y *= zv / (1.0f + __expf(-zv));
    }
    store_float((char*)vbase(p.out, b, h), p.out.dtype, pp * p.out.s[2], y);
  }
  if (L.active) store_state16<SDT, VEC>(p, sb, pp, n0, hv);
}

// Rows kernel for the model's decode call: state rows contiguous (row stride N) in 16-byte
// aligned (batch, head) slices, B and C bf16 with a contiguous d_state, dt, dt_bias, A and D
// constant within a head. 256 threads; lane (slot, blk) owns rows slot and slot + SLOTS, and in
// each row the 16-byte chunks blk, blk + BPR, ... (VPC = 16 / sizeof(state) values each), so that
// every load and store instruction of a wave covers whole consecutive rows. Every load of the lane
// (its state chunks, x, z, B, C, the head scalars) is issued before the first use of any of them,
// through per-(batch, head) buffer descriptors with the streaming state policy; the state goes
// back with the hardware round-to-nearest-even converts.
constexpr int SSM_ROWS = 2;

template <int SDT, int BPR_LOG2>
__global__ __launch_bounds__(256) void ssm_update_rows_kernel(SsmParams p) {
  constexpr int BPR = 1 << BPR_LOG2;
  constexpr uint32_t N = 16 * BPR;
  constexpr int SLOTS = 256 >> BPR_LOG2;
  constexpr int R = SSM_ROWS;
  constexpr uint32_t ES = SDT == LQ_F32 ? 4 : 2;
  constexpr int VPC = 16 / ES;     // state values per 16-byte chunk
  constexpr int NCH = 16 / VPC;    // chunks per lane and row
  const int h = blockIdx.y, b = blockIdx.z;
  const int blk = threadIdx.x & (BPR - 1);
  const int slot = threadIdx.x >> BPR_LOG2;
  const int P = p.P;
  const int row0 = blockIdx.x * (R * SLOTS);

  const auto rs = make_buf(vbase(p.st, b, h), (uint32_t)P * N * ES);
  const auto rx = make_buf(vbase(p.x, b, h), p.x_span);
  const auto rz = make_buf(vbase(p.z, b, h), p.z_span);  // span 0 without z: loads return 0
  u32x4_t sw[R][NCH];
  uint32_t xw[R], zw[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t pc = (uint32_t)min(row0 + r * SLOTS + slot, P - 1);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      sw[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rs, pc * N * ES + (j * BPR + blk) * 16u, 0,
                                                       STATE_LOAD_POLICY);
    }
    xw[r] = __builtin_amdgcn_raw_buffer_load_b32(rx, (pc * p.x_row_bytes) & ~3u, 0, 0);
    zw[r] = __builtin_amdgcn_raw_buffer_load_b32(rz, (pc * p.z_row_bytes) & ~3u, 0, 0);
  }
  // B and C at the lane's d_state positions: VPC bf16 values per chunk (16 or 8 bytes)
  const int grp = h / p.ratio;
  const auto rB = make_buf(vbase(p.B, b, grp), N * 2);
  const auto rC = make_buf(vbase(p.C, b, grp), N * 2);
  uint32_t bw[8], cw[8];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const uint32_t off = (uint32_t)(j * BPR + blk) * VPC * 2u;
    if constexpr (VPC == 8) {
      const u32x4_t vb = __builtin_amdgcn_raw_buffer_load_b128(rB, off, 0, 0);
      const u32x4_t vc = __builtin_amdgcn_raw_buffer_load_b128(rC, off, 0, 0);
      bw[4 * j] = vb.x; bw[4 * j + 1] = vb.y; bw[4 * j + 2] = vb.z; bw[4 * j + 3] = vb.w;
      cw[4 * j] = vc.x; cw[4 * j + 1] = vc.y; cw[4 * j + 2] = vc.z; cw[4 * j + 3] = vc.w;
    } else {
      const u32x2_t vb = __builtin_amdgcn_raw_buffer_load_b64(rB, off, 0, 0);
      const u32x2_t vc = __builtin_amdgcn_raw_buffer_load_b64(rC, off, 0, 0);
      bw[2 * j] = vb.x; bw[2 * j + 1] = vb.y;
      cw[2 * j] = vc.x; cw[2 * j + 1] = vc.y;
    }
  }
  const HeadScalars hs = head_scalars(p, b, h);
  float Bd[16], Cv[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    Bd[2 * i] = __uint_as_float(bw[i] << 16) * hs.dt;
    Bd[2 * i + 1] = __uint_as_float(bw[i] & 0xffff0000u) * hs.dt;
    Cv[2 * i] = __uint_as_float(cw[i] << 16);
    Cv[2 * i + 1] = __uint_as_float(cw[i] & 0xffff0000u);
  }
  const auto ro = make_buf(vbase(p.out, b, h), p.out_span);

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int pp = row0 + r * SLOTS + slot;
    const bool act = pp < P;
    const uint32_t pc = (uint32_t)min(pp, P - 1);
    const float xv = word_elem(xw[r], ((pc * p.x_row_bytes) & 2u) * 8u, p.x.dtype);
    float hv[16];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const uint32_t a[4] = {sw[r][j].x, sw[r][j].y, sw[r][j].z, sw[r][j].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if constexpr (SDT == LQ_F32) {
          hv[4 * j + w] = __uint_as_float(a[w]);
        } else {
          hv[8 * j + 2 * w] = word_elem(a[w], 0, SDT);
          hv[8 * j + 2 * w + 1] = word_elem(a[w], 16, SDT);
        }
      }
    }
    float ypart = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      hv[i] = fmaf(hv[i], hs.dA, Bd[i] * xv);
      ypart = fmaf(hv[i], Cv[i], ypart);
    }
    float y = row_sum<BPR_LOG2>(ypart);
    if (p.has_D) y += xv * hs.D;
    if (p.has_z) {
      const float zv = word_elem(zw[r], ((pc * p.z_row_bytes) & 2u) * 8u, p.z.dtype);
      y *= zv / (1.0f + __expf(-zv));
    }
    if (act && blk == 0) {
      const uint32_t oo = (uint32_t)pp * p.out_row_bytes;
      if (p.out.dtype == LQ_F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), ro, oo, 0, 0);
      } else if (p.out.dtype == LQ_BF16) {
        __builtin_amdgcn_raw_buffer_store_b16(float_to_bf16_bits(y), ro, oo, 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)y), ro, oo,
                                              0, 0);
      }
    }
    if (act) {
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        u32x4_t w;
        if constexpr (SDT == LQ_F32) {
          w = u32x4_t{__float_as_uint(hv[4 * j]), __float_as_uint(hv[4 * j + 1]),
                      __float_as_uint(hv[4 * j + 2]), __float_as_uint(hv[4 * j + 3])};
        } else {
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const f32x2_t v2{hv[8 * j + 2 * i], hv[8 * j + 2 * i + 1]};
            if constexpr (SDT == LQ_BF16) {
              o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v2, bf16x2_t));
            } else {
              o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v2, f16x2_t));
            }
          }
          w = u32x4_t{o[0], o[1], o[2], o[3]};
        }
        __builtin_amdgcn_raw_buffer_store_b128(w, rs, (uint32_t)pp * N * ES + (j * BPR + blk) * 16u,
                                               0, STATE_STORE_POLICY);
      }
    }
  }
}

template <int SDT>
static void launch_ssm_rows(const SsmParams& p, dim3 grid, hipStream_t st) {
  switch (p.vbpr_log2) {
    case 2: hipLaunchKernelGGL((ssm_update_rows_kernel<SDT, 2>), grid, dim3(256), 0, st, p); break;
    case 3: hipLaunchKernelGGL((ssm_update_rows_kernel<SDT, 3>), grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((ssm_update_rows_kernel<SDT, 4>), grid, dim3(256), 0, st, p); break;
  }
}

template <int SDT>
static void launch_ssm(const SsmParams& p, bool vec, bool bcvec, dim3 grid, hipStream_t st) {
  const dim3 block(256);
  if (vec && bcvec) {
    hipLaunchKernelGGL((ssm_update_kernel<SDT, true, true>), grid, block, 0, st, p);
  } else if (vec) {
    hipLaunchKernelGGL((ssm_update_kernel<SDT, true, false>), grid, block, 0, st, p);
  } else if (bcvec) {
    hipLaunchKernelGGL((ssm_update_kernel<SDT, false, true>), grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((ssm_update_kernel<SDT, false, false>), grid, block, 0, st, p);
  }
}

static int ssm_shape3(const lq_tensor* t, const char* name, int64_t a, int64_t b, int64_t c,
                      bool allow_null) {
  if (t == nullptr && allow_null) return LQ_OK;
  int rc;
  if ((rc = check_tensor(t, name, 3, true)) != LQ_OK) return rc;
  if (t->shape[0] != a || t->shape[1] != b || t->shape[2] != c) {
    return fail(LQ_ERR_INVALID_ARG, "%s must be [%lld, %lld, %lld]", name, (long long)a,
                (long long)b, (long long)c);
  }
  return LQ_OK;
}

static int ssm_shape2(const lq_tensor* t, const char* name, int64_t a, int64_t b) {
  if (t == nullptr) return LQ_OK;
  int rc;
  if ((rc = check_tensor(t, name, 2, true)) != LQ_OK) return rc;
  if (t->shape[0] != a || t->shape[1] != b) {
    return fail(LQ_ERR_INVALID_ARG, "%s must be [%lld, %lld]", name, (long long)a, (long long)b);
  }
  return LQ_OK;
}

// Lane offsets below the (batch, head) level are 32-bit: the span of dims >= first must fit.
static bool span32(const lq_tensor* t, int first, int64_t* bytes = nullptr) {
  if (t == nullptr) return true;
  int64_t span = 0;
  for (int i = 0; i < t->ndim; ++i) {
    if (t->stride[i] < 0) return false;
    if (i >= first && t->shape[i] > 0) span += (t->shape[i] - 1) * t->stride[i];
  }
  if (bytes != nullptr) *bytes = (span + 1) * dtype_size(t->dtype);
  return (span + 1) * dtype_size(t->dtype) < ((int64_t)1 << 31) - 64;
}

}  // namespace lq

using namespace lq;

extern "C" int lq_selective_state_update(const lq_tensor* state, const lq_tensor* x,
                                         const lq_tensor* dt, const lq_tensor* dt_bias,
                                         const lq_tensor* A, const lq_tensor* B,
                                         const lq_tensor* C, const lq_tensor* D,
                                         const lq_tensor* z, const lq_tensor* out,
                                         int dt_softplus, void* stream) {
  int rc;
  if ((rc = check_tensor(state, "state", 4, true)) != LQ_OK) return rc;
  const int64_t Bn = state->shape[0], H = state->shape[1], P = state->shape[2],
                N = state->shape[3];
  if (N % 16 != 0 || N / 16 > 64) {
    return fail(LQ_ERR_UNSUPPORTED, "state dim must be a multiple of 16 up to 1024, got %lld",
                (long long)N);
  }
  if ((rc = ssm_shape3(x, "x", Bn, H, P, false)) != LQ_OK) return rc;
  if ((rc = ssm_shape3(dt, "dt", Bn, H, P, false)) != LQ_OK) return rc;
  if ((rc = ssm_shape3(z, "z", Bn, H, P, true)) != LQ_OK) return rc;
  if ((rc = ssm_shape3(out, "out", Bn, H, P, false)) != LQ_OK) return rc;
  if ((rc = ssm_shape2(dt_bias, "dt_bias", H, P)) != LQ_OK) return rc;
  if ((rc = ssm_shape2(D, "D", H, P)) != LQ_OK) return rc;
  if ((rc = check_tensor(A, "A", 3, true)) != LQ_OK) return rc;
  if (A->shape[0] != H || A->shape[1] != P || A->shape[2] != N) {
    return fail(LQ_ERR_INVALID_ARG, "A must be [%lld, %lld, %lld]", (long long)H, (long long)P,
                (long long)N);
  }
  if ((rc = check_tensor(B, "B", 3, true)) != LQ_OK) return rc;
  if ((rc = check_tensor(C, "C", 3, true)) != LQ_OK) return rc;
  const int64_t G = B->shape[1];
  if (B->shape[0] != Bn || B->shape[2] != N || C->shape[0] != Bn || C->shape[1] != G ||
      C->shape[2] != N) {
    return fail(LQ_ERR_INVALID_ARG, "B and C must be [batch, ngroups, dstate]");
  }
  if (G <= 0 || H % G != 0) {
    return fail(LQ_ERR_INVALID_ARG, "nheads=%lld not divisible by ngroups=%lld", (long long)H,
                (long long)G);
  }
  if (Bn > 65535 || H > 65535) {
    return fail(LQ_ERR_UNSUPPORTED, "batch or heads exceed 65535");
  }
  if (Bn == 0 || H == 0 || P == 0) return LQ_OK;
  int64_t st_bytes = 0;
  const lq_tensor* lane_level[] = {x, dt, B, C, z, out};
  for (const lq_tensor* t : lane_level) {
    if (!span32(t, 2)) return fail(LQ_ERR_UNSUPPORTED, "tensor spans exceed 32-bit offsets");
  }
  if (!span32(state, 2, &st_bytes) || !span32(A, 1) || !span32(D, 1) || !span32(dt_bias, 1)) {
    return fail(LQ_ERR_UNSUPPORTED, "tensor spans exceed 32-bit offsets");
  }

  SsmParams p{};
  p.st = make_view(state);
  p.x = make_view(x);
  p.dt = make_view(dt);
  p.dtb = make_view(dt_bias);
  p.A = make_view(A);
  p.B = make_view(B);
  p.C = make_view(C);
  p.D = make_view(D);
  p.z = make_view(z);
  p.out = make_view(out);
  p.Bn = (int)Bn;
  p.H = (int)H;
  p.P = (int)P;
  p.N = (int)N;
  p.ratio = (int)(H / G);
  p.bpr = (int)(N / 16);
  p.vbpr_log2 = 0;
  while ((1 << p.vbpr_log2) < p.bpr) ++p.vbpr_log2;
  p.has_dtb = dt_bias != nullptr;
  p.has_D = D != nullptr;
  p.has_z = z != nullptr;
  p.softplus = dt_softplus != 0;
  p.a_row_const = A->stride[2] == 0;
  p.st_span = (uint32_t)((st_bytes + 15) & ~(int64_t)15);

  const int es = dtype_size(state->dtype);
  const bool vec = state->stride[3] == 1 && ((uintptr_t)state->data % 16) == 0 &&
                   (state->stride[0] * es) % 16 == 0 && (state->stride[1] * es) % 16 == 0 &&
                   (state->stride[2] * es) % 16 == 0;
  auto bcv = [](const lq_tensor* t) {
    return t->dtype == LQ_BF16 && t->stride[2] == 1 && ((uintptr_t)t->data & 15) == 0 &&
           t->stride[0] % 8 == 0 && t->stride[1] % 8 == 0;
  };
  const bool bcvec = bcv(B) && bcv(C);
  hipStream_t s = (hipStream_t)stream;
  const bool forced = diag(LQ_DIAG_SSM_FORCE_GENERIC);
  const int64_t lim = (int64_t)1 << 28;
  const bool rows_ok =
      !forced && vec && bcvec && (N == 64 || N == 128 || N == 256) && state->stride[2] == N &&
      dt->stride[2] == 0 && A->stride[1] == 0 && A->stride[2] == 0 &&
      (dt_bias == nullptr || dt_bias->stride[1] == 0) && (D == nullptr || D->stride[1] == 0) &&
      x->stride[2] >= 0 && out->stride[2] >= 0 && (z == nullptr || z->stride[2] >= 0) &&
      P * x->stride[2] < lim && P * out->stride[2] < lim && (z == nullptr || P * z->stride[2] < lim) &&
      P * N * es < ((int64_t)1 << 31);
  if (rows_ok) {
    auto row_bytes = [](const View& v) { return (uint32_t)(v.s[2] * dtype_size(v.dtype)); };
    auto span = [&](const View& v) {
      return (uint32_t)((((P - 1) * v.s[2] + 1) * dtype_size(v.dtype) + 3) & ~(int64_t)3);
    };
    p.x_row_bytes = row_bytes(p.x);
    p.x_span = span(p.x);
    p.out_row_bytes = row_bytes(p.out);
    p.out_span = span(p.out);
    if (p.has_z) {
      p.z_row_bytes = row_bytes(p.z);
      p.z_span = span(p.z);
    } else {  // a zero-span descriptor on x: its loads return 0 without reading memory
      p.z = p.x;
      p.z_row_bytes = 0;
      p.z_span = 0;
    }
    const View dt0{p.dt.data, p.dt.dtype, {0, 0, 0, 0}};
    if (!p.has_dtb) p.dtb = dt0;
    if (!p.has_D) p.D = dt0;
    const int rows = SSM_ROWS * (256 >> p.vbpr_log2);
    const dim3 rgrid((unsigned)((P + rows - 1) / rows), (unsigned)H, (unsigned)Bn);
    switch (state->dtype) {
      case LQ_BF16: launch_ssm_rows<LQ_BF16>(p, rgrid, s); break;
      case LQ_F16: launch_ssm_rows<LQ_F16>(p, rgrid, s); break;
      default: launch_ssm_rows<LQ_F32>(p, rgrid, s); break;
    }
    return check_launch("lq_selective_state_update");
  }
  if (diag(LQ_DIAG_SSM_REQUIRE_ROWS)) {  // tests: the call must take the row kernel
    return fail(LQ_ERR_INVALID_ARG,
                "LQ_SSM_REQUIRE_ROWS is set and this call's layout takes the general kernel");
  }
  const int64_t lanes = P << p.vbpr_log2;
  const dim3 grid((unsigned)((lanes + 255) / 256), (unsigned)H, (unsigned)Bn);
  switch (state->dtype) {
    case LQ_BF16: launch_ssm<LQ_BF16>(p, vec, bcvec, grid, s); break;
    case LQ_F16: launch_ssm<LQ_F16>(p, vec, bcvec, grid, s); break;
    default: launch_ssm<LQ_F32>(p, vec, bcvec, grid, s); break;
  }
  return check_launch("lq_selective_state_update");
}
