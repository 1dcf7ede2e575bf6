// INT4 KV pack: quantize new K or V tokens per group and write them into the packed cache.
//
// Replaces _pack_int4_kv_kernel (reference hybrid_quant/int4_8b_attention.py:32-111). Per group
// of g values along head_dim: absmax -> scale = max(absmax / 7, 1e-8) -> q = rint(x / scale)
// (IEEE division, round half to even) -> clamp [-8, 7] -> two's-complement nibbles, even d in the
// low nibble. int4_pack_lanes_kernel gives one lane to each output byte (dims 2j, 2j+1), so a
// group is g/2 adjacent lanes and its absmax a shuffle reduction; int4_pack_kernel (one thread
// per group) covers group sizes whose g/2 is not a power of two up to 64. Both kernels take up to
// two tensors (blockIdx.y picks one): lq_int4_pack_kv_pair packs a layer's K and V in one launch.
#include <algorithm>

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

// One launch over pair.pp[0 .. n-1] (n = 1 or 2), sized for the larger tensor.
int launch_pack(const PackPair& pair, int n, int group_size, hipStream_t s, const char* what) {
  int64_t bytes = 0, groups = 0;
  for (int i = 0; i < n; ++i) {
    bytes = std::max(bytes, pack_bytes(pair.pp[i]));
    groups = std::max(groups, pack_bytes(pair.pp[i]) * 2 / group_size);
  }
  if (bytes == 0) return LQ_OK;
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
