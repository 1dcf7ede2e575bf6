// Shared declarations of the INT4 decode-attention kernels.
#pragma once

#include <algorithm>

#include "lq_common.h"

namespace lq {

struct AttnParams {
  View q;  // strides of (b, h, d)
  const uint8_t* kp;
  const uint8_t* vp;
  int64_t kps[4], vps[4];
  const float* ks;
  const float* vs;
  int64_t kss[4], vss[4];
  const float* mask;  // NULL or [B, 1, 1, Lm] fp32 bias (batch and key strides used)
  int64_t mask_sb, mask_sk, mask_len;
  View out;  // strides of (b, h, d)
  float* ws_m;
  float* ws_l;
  float* ws_acc;
  int B, Hq, Hkv, D, g, nrep;
  int64_t S;
  int nsplit;     // workgroup splits along the keys
  int64_t chunk;  // keys per workgroup split
  float scale_sm; // log2(e) / sqrt(D)
  // fused pack (lq_int4_decode_attention_pack, MFMA path): the new token's K and V rows
  // [B, Hkv, D] (strides of b, h, d) are packed into cache row S - 1 inside the kernel
  View knew, vnew;
  int pack;
};

struct SplitPlan {
  int nsplit;
  int64_t chunk;
};

// fast path (int4_attention_mfma.hip)
bool fast_path_shape_ok(int64_t head_dim, int group_size, int64_t n_q_heads, int64_t n_kv_heads);
bool fast_path_ok(const AttnParams& p);
SplitPlan plan_fast(int64_t B, int64_t Hkv, int64_t S);
int launch_fast(const AttnParams& p, hipStream_t stream);

}  // namespace lq
