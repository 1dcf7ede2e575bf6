// INT4 KV pack: quantize new K or V tokens per group and write them into the packed cache.
//
// Replaces _pack_int4_kv_kernel (reference hybrid_quant/int4_8b_attention.py:32-111). Per group
// of g values along head_dim: absmax -> scale = max(absmax / 7, 1e-8) -> q = rint(x / scale)
// (IEEE division, round half to even) -> clamp [-8, 7] -> two's-complement nibbles, even d in the
// low nibble. int4_pack_lanes_kernel gives one lane to each output byte (dims 2j, 2j+1), so a
// group is g/2 adjacent lanes and its absmax a shuffle reduction; int4_pack_kernel (one thread
// per group) covers group sizes whose g/2 is not a power of two up to 64. int4_pack_rows_kernel
// takes the common layout (contiguous rows, 16-byte aligned, g a multiple of 8): one lane per 8
// values of each of 4 rows (16- or 32-byte loads issued together, 4-byte stores), g/8 lanes per
// group, and the division by the scale done as a product with the reciprocal wherever that
// provably gives the same level.
// All kernels take up to two tensors (blockIdx.y picks one): lq_int4_pack_kv_pair packs a layer's
// K and V in one launch.
#include <algorithm>
#include <type_traits>

#include "int4_quant.h"
#include "lq_common.h"

namespace lq {

struct PackParams {
  View x;  // [B, Hkv, T, D]
  uint8_t* packed;
  int64_t ps[4];  // [B, Hkv, cap, D/2]
  float* scale;
  int64_t ss[4];  // [B, Hkv, cap, D/g]
  const int64_t* positions;  // NULL: token t goes to row fixed_pos + t
  int64_t pos_stride;
  int64_t fixed_pos;
  int B, H, T, D, g;
  int64_t cap;
};

// The tensors of one launch: pp[blockIdx.y] (one entry used by lq_int4_pack_kv).
struct PackPair {
  PackParams pp[2];
};

// One lane per packed byte; GH = g/2 lanes per group (a power of two <= 64, so groups never
// straddle a wave). Lane offsets are 32-bit (the host checks the element count).
template <int GH>
__global__ __launch_bounds__(256) void int4_pack_lanes_kernel(PackPair pair) {
  const PackParams& p = pair.pp[blockIdx.y];
  const int half = p.D >> 1;
  const int total = p.B * p.H * p.T * half;
  if (total == 0) return;  // an empty tensor of a pair
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const bool in = gid < total;
  const int g2 = in ? gid : total - 1;  // whole trailing groups only; they store nothing
  const int j = g2 % half;
  const int row = g2 / half;
  const int t = row % p.T;
  const int bh = row / p.T;
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int64_t xrow = b * p.x.s[0] + h * p.x.s[1] + t * p.x.s[2];
  const float v0 = load_float(p.x.data, p.x.dtype, xrow + (2 * j) * p.x.s[3]);
  const float v1 = load_float(p.x.data, p.x.dtype, xrow + (2 * j + 1) * p.x.s[3]);
  float scale;
  const uint32_t byte = int4_quantize_pair<GH>(v0, v1, scale);
  const int64_t pos = p.positions != nullptr ? p.positions[t * p.pos_stride] : p.fixed_pos + t;
  if (!in || pos < 0 || pos >= p.cap) return;
  p.packed[b * p.ps[0] + h * p.ps[1] + pos * p.ps[2] + j * p.ps[3]] = (uint8_t)byte;
  if ((j & (GH - 1)) == 0) {
    p.scale[b * p.ss[0] + h * p.ss[1] + pos * p.ss[2] + (j / GH) * p.ss[3]] = scale;
  }
}

// 8 values of a token row as raw words (bf16 / fp16: one 16-byte load; fp32: two).
template <int DT>
struct Raw8 {
  uint4 a, c;
};

template <int DT>
__device__ __forceinline__ Raw8<DT> load8(const void* base, int64_t e) {
  Raw8<DT> r;
  if constexpr (DT == LQ_F32) {
    r.a = *(const uint4*)((const float*)base + e);
    r.c = *(const uint4*)((const float*)base + e + 4);
  } else {
    r.a = *(const uint4*)((const uint16_t*)base + e);
  }
  return r;
}

template <int DT>
__device__ __forceinline__ void decode8(const Raw8<DT>& r, float (&v)[8]) {
  if constexpr (DT == LQ_F32) {
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
  } else {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == LQ_BF16) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)w[i]);
        v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
      }
    }
  }
}

// The packed nibbles of NV values of one group (NV / 8 words, two's-complement levels, the even
// value in the low nibble), equal to clamp(rint(RN(x / scale)), -8, 7) of the IEEE quotient bit
// for bit. With y = RN(x * rcp(scale)) (v_rcp_f32 within 1 ulp), |y - RN(x / scale)| <=
// |x / scale| * (2^-23 + 2^-23 + 2^-24) <= 2^-19 for |x / scale| <= 8, so when y lies more than
// 2^-17 from every half-integer both round to the same integer (no half-integer lies between
// them); a lane with a value closer than that (or a non-finite one, or a non-finite scale)
// recomputes its levels with the IEEE division. t = RN(y + 1.5 * 2^23) is y rounded to an integer
// k (ties to even) held in the low mantissa bits as k + 2^22, so its low 4 bits are k's
// two's-complement nibble; |k| <= 7 here because |x| <= absmax and scale >= absmax / 7 rounded.
template <int NV>
__device__ __forceinline__ void pack_levels(const float (&v)[NV], float scale,
                                            uint32_t (&words)[NV / 8]) {
  constexpr float C = 12582912.0f;  // 1.5 * 2^23
  const float rcp = __builtin_amdgcn_rcpf(scale);
  float t[NV];
  bool exact = !(scale < INFINITY);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const float y = v[i] * rcp;
    t[i] = y + C;
    exact |= !(fabsf(y - (t[i] - C)) < 0.5f - 0x1p-17f);
  }
  if (exact) {  // rare
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int q = min(max((int)rintf(v[i] / scale), -8), 7);
      t[i] = (float)q + C;
    }
  }
#pragma unroll
  for (int w = 0; w < NV / 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= (__float_as_uint(t[8 * w + i]) & 15u) << (4 * i);
    words[w] = word;
  }
}

// The 4 packed bytes of 8 values whose group spans L8 adjacent lanes (every lane of the wave
// active), and the group's scale (levels as in pack_levels).
template <int L8>
__device__ __forceinline__ uint32_t quantize8(const float (&v)[8], float& scale) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int o = L8 >> 1; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  scale = fmaxf(amax / 7.0f, 1.0e-8f);
  uint32_t word[1];
  pack_levels<8>(v, scale, word);
  return word[0];
}

// One lane per quantisation group of G values (16, 32 or 64) of a token row: G / 8 loads of 16
// bytes (bf16 / fp16; twice that for fp32) issued together, the group's absmax within the lane,
// and its G / 2 packed bytes written as 8- or 16-byte stores, its scale as one word: a wave reads
// and writes whole consecutive rows. Rows contiguous (x stride 1 along head_dim, 16-byte aligned;
// packed rows 16-byte aligned, or 8-byte for G = 16). Grid (lanes of one (batch, head) slice /
// 256, B * H, tensors); head_dim / G = 2^lr_log2 lanes per token row.
template <int G, int DT>
__global__ __launch_bounds__(256) void int4_pack_groups_kernel(PackPair pair, int lr_log2) {
  const PackParams& p = pair.pp[blockIdx.z];
  const int total = p.T << lr_log2;
  if (total == 0 || (int)blockIdx.y >= p.B * p.H) return;  // an empty or smaller tensor
  const int gid = (int)blockIdx.x * 256 + (int)threadIdx.x;
  const int g2 = min(gid, total - 1);
  const int k = g2 & ((1 << lr_log2) - 1);  // group within the row
  const int t = g2 >> lr_log2;
  const int b = (int)blockIdx.y / p.H;
  const int h = (int)blockIdx.y - b * p.H;
  const int64_t xe = b * p.x.s[0] + h * p.x.s[1] + t * p.x.s[2] + G * k;
  constexpr int NL = G / 8;
  Raw8<DT> raw[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) raw[i] = load8<DT>(p.x.data, xe + 8 * i);
  float v[G];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    float w[8];
    decode8<DT>(raw[i], w);
#pragma unroll
    for (int u = 0; u < 8; ++u) v[8 * i + u] = w[u];
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float scale = fmaxf(amax / 7.0f, 1.0e-8f);
  uint32_t words[G / 8];
  pack_levels<G>(v, scale, words);
  if (gid >= total) return;
  const int64_t pos = p.positions != nullptr ? p.positions[t * p.pos_stride] : p.fixed_pos + t;
  if (pos < 0 || pos >= p.cap) return;
  uint8_t* dst = p.packed + b * p.ps[0] + h * p.ps[1] + pos * p.ps[2] + (G / 2) * k;
  if constexpr (G == 16) {
    *(uint2*)dst = make_uint2(words[0], words[1]);
  } else {
#pragma unroll
    for (int w = 0; w < G / 32; ++w) {
      *(uint4*)(dst + 16 * w) = make_uint4(words[4 * w], words[4 * w + 1], words[4 * w + 2],
                                           words[4 * w + 3]);
    }
  }
  p.scale[b * p.ss[0] + h * p.ss[1] + pos * p.ss[2] + k * p.ss[3]] = scale;
}

// One lane per 8 values of a token row (dims 8j .. 8j + 7 -> packed bytes 4j .. 4j + 3) in each
// of R rows, L8 = g/8 lanes per group (a power of two <= 64: a group never straddles a wave); rows
// contiguous (x stride 1 along head_dim, 16-byte aligned; packed bytes 4-byte aligned). The R
// rows' loads are issued together. Grid (rows of one (batch, head) slice / (R * 256 / lanes per
// row), B * H, tensors); head_dim / 8 = 2^lr_log2 lanes per token row.
template <int L8, int DT, int R>
__global__ __launch_bounds__(256) void int4_pack_rows_kernel(PackPair pair, int lr_log2) {
  const PackParams& p = pair.pp[blockIdx.z];
  if (p.T == 0 || (int)blockIdx.y >= p.B * p.H) return;  // an empty or smaller tensor
  const int rows_step = 256 >> lr_log2;                    // rows per r
  const int j = threadIdx.x & ((1 << lr_log2) - 1);
  const int t0 = (int)blockIdx.x * R * rows_step + ((int)threadIdx.x >> lr_log2);
  const int b = (int)blockIdx.y / p.H;
  const int h = (int)blockIdx.y - b * p.H;
  const int64_t xb = b * p.x.s[0] + h * p.x.s[1] + 8 * j;
  Raw8<DT> raw[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = min(t0 + r * rows_step, p.T - 1);  // whole groups share a row
    raw[r] = load8<DT>(p.x.data, xb + t * p.x.s[2]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = t0 + r * rows_step;
    float v[8];
    decode8<DT>(raw[r], v);
    float scale;
    const uint32_t word = quantize8<L8>(v, scale);
    if (t >= p.T) continue;
    const int64_t pos = p.positions != nullptr ? p.positions[t * p.pos_stride] : p.fixed_pos + t;
    if (pos < 0 || pos >= p.cap) continue;
    *(uint32_t*)(p.packed + b * p.ps[0] + h * p.ps[1] + pos * p.ps[2] + 4 * j) = word;
    if ((j & (L8 - 1)) == 0) {
      p.scale[b * p.ss[0] + h * p.ss[1] + pos * p.ss[2] + (j / L8) * p.ss[3]] = scale;
    }
  }
}

__global__ __launch_bounds__(256) void int4_pack_kernel(PackPair pair) {
  const PackParams& p = pair.pp[blockIdx.y];
  const int groups = p.D / p.g;
  const int64_t total = (int64_t)p.B * p.H * p.T * groups;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= total) return;
  const int grp = (int)(gid % groups);
  int64_t r = gid / groups;
  const int t = (int)(r % p.T);
  r /= p.T;
  const int h = (int)(r % p.H);
  const int b = (int)(r / p.H);
  const int64_t pos = p.positions != nullptr ? p.positions[t * p.pos_stride] : p.fixed_pos + t;
  if (pos < 0 || pos >= p.cap) return;

  const int64_t xrow = b * p.x.s[0] + h * p.x.s[1] + t * p.x.s[2];
  const int d0 = grp * p.g;
  float amax = 0.0f;
  for (int i = 0; i < p.g; ++i) {
    amax = fmaxf(amax, fabsf(load_float(p.x.data, p.x.dtype, xrow + (d0 + i) * p.x.s[3])));
  }
  const float scale = fmaxf(amax / 7.0f, 1.0e-8f);

  uint8_t* dst = p.packed + b * p.ps[0] + h * p.ps[1] + pos * p.ps[2];
  for (int i = 0; i < p.g; i += 2) {
    const float v0 = load_float(p.x.data, p.x.dtype, xrow + (d0 + i) * p.x.s[3]);
    const float v1 = load_float(p.x.data, p.x.dtype, xrow + (d0 + i + 1) * p.x.s[3]);
    int q0 = (int)rintf(v0 / scale);
    int q1 = (int)rintf(v1 / scale);
    q0 = min(max(q0, -8), 7);
    q1 = min(max(q1, -8), 7);
    dst[((d0 + i) >> 1) * p.ps[3]] = (uint8_t)(((q1 & 15) << 4) | (q0 & 15));
  }
  p.scale[b * p.ss[0] + h * p.ss[1] + pos * p.ss[2] + grp * p.ss[3]] = scale;
}

}  // namespace lq

using namespace lq;

namespace {

// Validate one (x, packed, scale) triple against positions (a device tensor, or NULL for the
// rows fixed_pos, fixed_pos + 1, ...) and fill its launch parameters.
int make_pack_params(const lq_tensor* x, const lq_tensor* packed, const lq_tensor* scale,
                     const lq_tensor* positions, int group_size, PackParams& p,
                     int64_t fixed_pos = 0) {
  int rc;
  if ((rc = check_tensor(x, "x", 4, true)) != LQ_OK) return rc;
  if ((rc = check_tensor(packed, "packed", 4, false, LQ_U8)) != LQ_OK) return rc;
  if ((rc = check_tensor(scale, "scale", 4, false, LQ_F32)) != LQ_OK) return rc;
  if (positions != nullptr &&
      (rc = check_tensor(positions, "positions", 1, false, LQ_I64)) != LQ_OK) {
    return rc;
  }
  const int64_t B = x->shape[0], H = x->shape[1], T = x->shape[2], D = x->shape[3];
  if (group_size <= 0 || group_size % 2 != 0) {
    return fail(LQ_ERR_INVALID_ARG, "group_size=%d must be even for INT4 packing", group_size);
  }
  if (D % group_size != 0) {
    return fail(LQ_ERR_INVALID_ARG, "head_dim=%lld must be divisible by group_size=%d",
                (long long)D, group_size);
  }
  const int64_t cap = packed->shape[2];
  if (packed->shape[0] != B || packed->shape[1] != H || packed->shape[3] != D / 2) {
    return fail(LQ_ERR_INVALID_ARG, "packed must be [%lld, %lld, cap, %lld]", (long long)B,
                (long long)H, (long long)(D / 2));
  }
  if (scale->shape[0] != B || scale->shape[1] != H || scale->shape[2] != cap ||
      scale->shape[3] != D / group_size) {
    return fail(LQ_ERR_INVALID_ARG, "scale must be [%lld, %lld, %lld, %lld]", (long long)B,
                (long long)H, (long long)cap, (long long)(D / group_size));
  }
  if (positions != nullptr && positions->shape[0] != T) {
    return fail(LQ_ERR_INVALID_ARG, "positions has %lld entries for q_len=%lld",
                (long long)positions->shape[0], (long long)T);
  }
  if (positions == nullptr && (fixed_pos < 0 || fixed_pos + T > cap)) {
    return fail(LQ_ERR_INVALID_ARG, "rows %lld .. %lld outside the cache capacity %lld",
                (long long)fixed_pos, (long long)(fixed_pos + T - 1), (long long)cap);
  }
  p = PackParams{};
  p.x = make_view(x);
  p.packed = (uint8_t*)packed->data;
  p.scale = (float*)scale->data;
  for (int i = 0; i < 4; ++i) {
    p.ps[i] = packed->stride[i];
    p.ss[i] = scale->stride[i];
  }
  p.positions = positions != nullptr ? (const int64_t*)positions->data : nullptr;
  p.pos_stride = positions != nullptr ? positions->stride[0] : 0;
  p.fixed_pos = fixed_pos;
  p.B = (int)B;
  p.H = (int)H;
  p.T = (int)T;
  p.D = (int)D;
  p.g = group_size;
  p.cap = cap;
  return LQ_OK;
}

int64_t pack_bytes(const PackParams& p) { return (int64_t)p.B * p.H * p.T * (p.D / 2); }

// int4_pack_groups_kernel's layout: g of 16, 32 or 64 and head_dim / g a power of two, the row
// kernel's layout otherwise, and packed rows aligned to the lane's stores (16 bytes; 8 for g = 16).
bool rows_layout_ok(const PackPair& pair, int n, int group_size);
bool groups_layout_ok(const PackPair& pair, int n, int group_size) {
  if (group_size != 16 && group_size != 32 && group_size != 64) return false;
  if (!rows_layout_ok(pair, n, group_size)) return false;
  const int al = group_size == 16 ? 8 : 16;
  for (int i = 0; i < n; ++i) {
    const PackParams& p = pair.pp[i];
    const int lanes_row = p.D / group_size;
    if (p.D % group_size != 0 || (lanes_row & (lanes_row - 1)) != 0) return false;
    if (((uintptr_t)p.packed % al) != 0) return false;
    for (int d = 0; d < 3; ++d) {
      if (p.ps[d] % al != 0) return false;
    }
  }
  return true;
}

// int4_pack_rows_kernel's layout, for every tensor of the launch: the same dtype (bf16, fp16 or
// fp32) and head_dim; head_dim / 8 and g / 8 powers of two (g / 8 <= 64); x contiguous along
// head_dim with 16-byte aligned rows; packed bytes contiguous with 4-byte aligned rows.
bool rows_layout_ok(const PackPair& pair, int n, int group_size) {
  if (group_size % 8 != 0) return false;
  const int l8 = group_size / 8;
  if (l8 > 64 || (l8 & (l8 - 1)) != 0) return false;
  for (int i = 0; i < n; ++i) {
    const PackParams& p = pair.pp[i];
    if (p.x.dtype != pair.pp[0].x.dtype) return false;
    if (p.x.dtype != LQ_BF16 && p.x.dtype != LQ_F16 && p.x.dtype != LQ_F32) return false;
    const int lanes_row = p.D / 8;
    if (p.D % 8 != 0 || lanes_row != pair.pp[0].D / 8 || (lanes_row & (lanes_row - 1)) != 0) {
      return false;
    }
    if (p.x.s[3] != 1) return false;
    const int64_t es = p.x.dtype == LQ_F32 ? 4 : 2;
    if (((uintptr_t)p.x.data % 16) != 0) return false;
    for (int d = 0; d < 3; ++d) {
      if ((p.x.s[d] * es) % 16 != 0) return false;
    }
    if (p.ps[3] != 1 || ((uintptr_t)p.packed % 4) != 0) return false;
    for (int d = 0; d < 3; ++d) {
      if (p.ps[d] % 4 != 0) return false;
    }
  }
  return true;
}

// One launch over pair.pp[0 .. n-1] (n = 1 or 2), sized for the larger tensor.
int launch_pack(const PackPair& pair, int n, int group_size, hipStream_t s, const char* what) {
  int64_t bytes = 0, groups = 0;
  for (int i = 0; i < n; ++i) {
    bytes = std::max(bytes, pack_bytes(pair.pp[i]));
    groups = std::max(groups, pack_bytes(pair.pp[i]) * 2 / group_size);
  }
  if (bytes == 0) return LQ_OK;
  int64_t slice_rows = 0, slices = 0;
  for (int i = 0; i < n; ++i) {
    slice_rows = std::max(slice_rows, (int64_t)pair.pp[i].T);
    slices = std::max(slices, (int64_t)pair.pp[i].B * pair.pp[i].H);
  }
  // The per-slice grids of the group and row kernels fit prompts (many tokens per (batch, head));
  // for a few tokens per slice (a decode token) most of their lanes would idle, and the
  // one-lane-per-byte kernel's flat grid fills the waves instead.
  const bool many_rows = slice_rows * (pair.pp[0].D / 8) >= 256;
  if (many_rows && groups_layout_ok(pair, n, group_size) &&
      slice_rows * (pair.pp[0].D / group_size) < ((int64_t)1 << 31) - 256 && slices <= 65535) {
    const int lr_log2 = __builtin_ctz((unsigned)(pair.pp[0].D / group_size));
    const int64_t lanes = slice_rows << lr_log2;
    const dim3 grid((unsigned)((lanes + 255) / 256), (unsigned)slices, (unsigned)n);
    const int dt = pair.pp[0].x.dtype;
    auto go = [&](auto gv) {
      constexpr int GV = decltype(gv)::value;
      if (dt == LQ_BF16) {
        hipLaunchKernelGGL((int4_pack_groups_kernel<GV, LQ_BF16>), grid, dim3(256), 0, s, pair,
                           lr_log2);
      } else if (dt == LQ_F16) {
        hipLaunchKernelGGL((int4_pack_groups_kernel<GV, LQ_F16>), grid, dim3(256), 0, s, pair,
                           lr_log2);
      } else {
        hipLaunchKernelGGL((int4_pack_groups_kernel<GV, LQ_F32>), grid, dim3(256), 0, s, pair,
                           lr_log2);
      }
    };
    if (group_size == 16) go(std::integral_constant<int, 16>{});
    else if (group_size == 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
    return check_launch(what);
  }
  constexpr int RROWS = 4;  // rows per lane
  if (many_rows && rows_layout_ok(pair, n, group_size) &&
      slice_rows * (pair.pp[0].D / 8) < ((int64_t)1 << 31) && slices <= 65535 &&
      pair.pp[0].D / 8 <= 256) {
    const int lr_log2 = __builtin_ctz((unsigned)(pair.pp[0].D / 8));
    const int64_t rows_block = (int64_t)RROWS * (256 >> lr_log2);
    const dim3 grid((unsigned)((slice_rows + rows_block - 1) / rows_block), (unsigned)slices,
                    (unsigned)n);
    const int dt = pair.pp[0].x.dtype;
    bool ok = true;
    auto go = [&](auto l8) {
      constexpr int L8 = decltype(l8)::value;
      if (dt == LQ_BF16) {
        hipLaunchKernelGGL((int4_pack_rows_kernel<L8, LQ_BF16, RROWS>), grid, dim3(256), 0, s,
                           pair, lr_log2);
      } else if (dt == LQ_F16) {
        hipLaunchKernelGGL((int4_pack_rows_kernel<L8, LQ_F16, RROWS>), grid, dim3(256), 0, s,
                           pair, lr_log2);
      } else {
        hipLaunchKernelGGL((int4_pack_rows_kernel<L8, LQ_F32, RROWS>), grid, dim3(256), 0, s,
                           pair, lr_log2);
      }
    };
    switch (group_size / 8) {
      case 1: go(std::integral_constant<int, 1>{}); break;
      case 2: go(std::integral_constant<int, 2>{}); break;
      case 4: go(std::integral_constant<int, 4>{}); break;
      case 8: go(std::integral_constant<int, 8>{}); break;
      case 16: go(std::integral_constant<int, 16>{}); break;
      case 32: go(std::integral_constant<int, 32>{}); break;
      case 64: go(std::integral_constant<int, 64>{}); break;
      default: ok = false; break;
    }
    if (ok) return check_launch(what);
  }
  const int gh = group_size / 2;
  if (gh <= 64 && (gh & (gh - 1)) == 0 && bytes < ((int64_t)1 << 31) - 256) {
    const dim3 grid((unsigned)((bytes + 255) / 256), (unsigned)n);
    switch (gh) {
      case 1: hipLaunchKernelGGL(int4_pack_lanes_kernel<1>, grid, dim3(256), 0, s, pair); break;
      case 2: hipLaunchKernelGGL(int4_pack_lanes_kernel<2>, grid, dim3(256), 0, s, pair); break;
      case 4: hipLaunchKernelGGL(int4_pack_lanes_kernel<4>, grid, dim3(256), 0, s, pair); break;
      case 8: hipLaunchKernelGGL(int4_pack_lanes_kernel<8>, grid, dim3(256), 0, s, pair); break;
      case 16: hipLaunchKernelGGL(int4_pack_lanes_kernel<16>, grid, dim3(256), 0, s, pair); break;
      case 32: hipLaunchKernelGGL(int4_pack_lanes_kernel<32>, grid, dim3(256), 0, s, pair); break;
      default: hipLaunchKernelGGL(int4_pack_lanes_kernel<64>, grid, dim3(256), 0, s, pair); break;
    }
    return check_launch(what);
  }
  const int threads = 256;
  const int64_t blocks = (groups + threads - 1) / threads;
  hipLaunchKernelGGL(int4_pack_kernel, dim3((unsigned)blocks, (unsigned)n), dim3(threads), 0, s,
                     pair);
  return check_launch(what);
}

}  // namespace

extern "C" int lq_int4_pack_kv(const lq_tensor* x, const lq_tensor* packed,
                               const lq_tensor* scale, const lq_tensor* positions,
                               int group_size, void* stream) {
  PackPair pair{};
  int rc;
  if ((rc = make_pack_params(x, packed, scale, positions, group_size, pair.pp[0])) != LQ_OK) {
    return rc;
  }
  return launch_pack(pair, 1, group_size, (hipStream_t)stream, "lq_int4_pack_kv");
}

extern "C" int lq_int4_pack_kv_pair(const lq_tensor* k, const lq_tensor* v,
                                    const lq_tensor* k_packed, const lq_tensor* v_packed,
                                    const lq_tensor* k_scale, const lq_tensor* v_scale,
                                    const lq_tensor* positions, int group_size, void* stream) {
  PackPair pair{};
  int rc;
  if ((rc = make_pack_params(k, k_packed, k_scale, positions, group_size, pair.pp[0])) != LQ_OK) {
    return rc;
  }
  if ((rc = make_pack_params(v, v_packed, v_scale, positions, group_size, pair.pp[1])) != LQ_OK) {
    return rc;
  }
  return launch_pack(pair, 2, group_size, (hipStream_t)stream, "lq_int4_pack_kv_pair");
}

namespace lq {

int pack_pair_at(const lq_tensor* k, const lq_tensor* v, const lq_tensor* k_packed,
                 const lq_tensor* v_packed, const lq_tensor* k_scale, const lq_tensor* v_scale,
                 int64_t row, int group_size, bool launch, hipStream_t stream, const char* what) {
  PackPair pair{};
  int rc;
  if ((rc = make_pack_params(k, k_packed, k_scale, nullptr, group_size, pair.pp[0], row)) != LQ_OK) {
    return rc;
  }
  if ((rc = make_pack_params(v, v_packed, v_scale, nullptr, group_size, pair.pp[1], row)) != LQ_OK) {
    return rc;
  }
  return launch ? launch_pack(pair, 2, group_size, stream, what) : LQ_OK;
}

}  // namespace lq
