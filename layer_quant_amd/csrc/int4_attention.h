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
  uint32_t* ws_cnt;  // arrival counters of the (batch, KV head) units (fold)
  int fold;          // the fast kernel merges its own splits (LQ_DIAG_ATTN_FOLD_MERGE)
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

// Split-K workspace layout: arrival counters in a fixed area at the start (so that every shape
// finds them at the same place; zero before a workspace's first use, left zero by every call),
// then the partials m [slots], l [slots], acc [slots][D], each array 256-byte aligned.
constexpr int ARRIVAL_UNITS = 16384;  // (batch, KV head) units a folded merge can count
constexpr size_t ARRIVAL_BYTES = (size_t)ARRIVAL_UNITS * 4;
static_assert(ARRIVAL_BYTES == LQ_DECODE_ATTENTION_COUNTER_BYTES, "header and kernels agree");

// fast path (int4_attention_mfma.hip)
bool fast_fold_fits(int nrep, int nsplit);
bool fast_path_shape_ok(int64_t head_dim, int group_size, int64_t n_q_heads, int64_t n_kv_heads);
bool fast_path_ok(const AttnParams& p);
SplitPlan plan_fast(int64_t B, int64_t Hkv, int64_t S);
int launch_fast(const AttnParams& p, hipStream_t stream);

}  // namespace lq
