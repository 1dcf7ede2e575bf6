// q_len = 1 GQA decode attention over the packed INT4 KV cache.
//
// Replaces _int4_decode_attention_kernel (reference hybrid_quant/int4_8b_attention.py:254-402).
// Two kernels share one split-K plan and one merge:
//   * attn_fast_kernel (int4_attention_mfma.hip): head_dim 128, group 32/64/128, all query heads
//     of a KV head in one MFMA tile; every KV byte is read once per (batch, KV head).
//   * attn_generic_kernel (here): any even group dividing any head_dim <= 512, one wave per
//     (batch, query head, split), fp32 VALU throughout.
// Scores follow the reference: s_n = (q . k_n) * log2(e)/sqrt(D) (+ mask_n), exp2-domain online
// softmax; keys at or beyond the mask length get -inf. Splits write (m, l, acc[D]) partials into
// the caller's workspace and attn_merge_kernel merges them; a single split writes out directly.
// With LQ_DIAG_ATTN_FOLD_MERGE the MFMA kernel's last workgroup of each (batch, KV head) merges
// them instead (counted by arrival counters at the start of the workspace): one launch, but at
// batch 1 the kernel grows by more than the merge launch takes.
// lq_int4_decode_attention_pack first packs the new token into cache row seq_len - 1 (the
// reference's _pack_kv_into_cache at :477-515): inside attn_fast_kernel on the MFMA path, by the
// pack kernel before the generic one otherwise.
#include <math.h>

#include <atomic>
#include <mutex>

#include "int4_attention.h"
#include "int4_quant.h"

namespace lq {

constexpr int GEN_MAX_D = 512;

__global__ __launch_bounds__(64) void attn_generic_kernel(AttnParams p) {
  __shared__ float q_s[GEN_MAX_D];
  __shared__ float p_s[64];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int split = blockIdx.y;
  const int b = bh / p.Hq;
  const int qh = bh - b * p.Hq;
  const int kvh = qh / p.nrep;
  const int64_t t0 = (int64_t)split * p.chunk;
  const int64_t t1 = min(p.S, t0 + p.chunk);
  const int D = p.D;
  const int g = p.g;

  for (int d = lane; d < D; d += 64) {
    q_s[d] = load_float(p.q.data, p.q.dtype, b * p.q.s[0] + qh * p.q.s[1] + d * p.q.s[2]);
  }
  __syncthreads();

  const uint8_t* kbase = p.kp + b * p.kps[0] + kvh * p.kps[1];
  const uint8_t* vbase = p.vp + b * p.vps[0] + kvh * p.vps[1];
  const float* ksbase = p.ks + b * p.kss[0] + kvh * p.kss[1];
  const float* vsbase = p.vs + b * p.vss[0] + kvh * p.vss[1];
  const int groups = D / g;

  float m = -INFINITY;
  float l = 0.0f;
  float acc[GEN_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < GEN_MAX_D / 64; ++i) acc[i] = 0.0f;

  for (int64_t start = t0; start < t1; start += 64) {
    const int64_t n = start + lane;
    float s = -INFINITY;
    if (n < t1) {
      const uint8_t* kr = kbase + n * p.kps[2];
      const float* ksr = ksbase + n * p.kss[2];
      float tot = 0.0f;
      for (int gi = 0; gi < groups; ++gi) {
        float part = 0.0f;
        for (int d = gi * g; d < (gi + 1) * g; d += 2) {
          const int byte = kr[(d >> 1) * p.kps[3]];
          int lo = byte & 15;
          int hi = (byte >> 4) & 15;
          lo = lo >= 8 ? lo - 16 : lo;
          hi = hi >= 8 ? hi - 16 : hi;
          part += q_s[d] * (float)lo + q_s[d + 1] * (float)hi;
        }
        tot += part * ksr[gi * p.kss[3]];
      }
      s = tot * p.scale_sm;
      if (p.mask != nullptr) {
        s += (n < p.mask_len) ? p.mask[b * p.mask_sb + n * p.mask_sk] : -INFINITY;
      }
    }
    const float mt = group_max<64>(s);
    const float m_new = fmaxf(m, mt);
    const float alpha = (m_new == -INFINITY) ? 1.0f : exp2f(m - m_new);
    const float pn = (s == -INFINITY) ? 0.0f : exp2f(s - m_new);
    l = l * alpha + group_sum<64>(pn);
    p_s[lane] = pn;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GEN_MAX_D / 64; ++i) acc[i] *= alpha;
    const int cnt = (int)min((int64_t)64, t1 - start);
    for (int j = 0; j < cnt; ++j) {
      const float pj = p_s[j];
      const uint8_t* vr = vbase + (start + j) * p.vps[2];
      const float* vsr = vsbase + (start + j) * p.vss[2];
#pragma unroll
      for (int i = 0; i < GEN_MAX_D / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < D) {
          const int byte = vr[(d >> 1) * p.vps[3]];
          int nib = (d & 1) ? ((byte >> 4) & 15) : (byte & 15);
          nib = nib >= 8 ? nib - 16 : nib;
          acc[i] += pj * ((float)nib * vsr[(d / g) * p.vss[3]]);
        }
      }
    }
    __syncthreads();
    m = m_new;
  }

  if (p.nsplit == 1) {
#pragma unroll
    for (int i = 0; i < GEN_MAX_D / 64; ++i) {
      const int d = lane + 64 * i;
      if (d < D) store_float(p.out.data, p.out.dtype, b * p.out.s[0] + qh * p.out.s[1] + d * p.out.s[2], acc[i] / l);
    }
  } else {
    const int64_t slot = (int64_t)bh * p.nsplit + split;
    if (lane == 0) {
      p.ws_m[slot] = m;
      p.ws_l[slot] = l;
    }
#pragma unroll
    for (int i = 0; i < GEN_MAX_D / 64; ++i) {
      const int d = lane + 64 * i;
      if (d < D) p.ws_acc[slot * D + d] = acc[i];
    }
  }
}

// Combines the split partials of one (batch, query head): M = max m_s, w_s = 2^(m_s - M),
// out = sum w_s acc_s / sum w_s l_s. A split with m_s = -inf (all keys masked) has weight 0.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One 256-thread workgroup per (batch, query head), so that every split's partial row is loaded
// in parallel (a single wave walking the splits one after another paid a memory round trip per
// few splits, which dominated small batches at long contexts): M = max_s m_s and
// L = sum_s 2^(m_s - M) l_s by block reductions, then thread (g, d) sums 2^(m_s - M) acc_s[d] over
// the splits s = g mod G (G = 256 / D split groups for D <= 256; each thread takes two dims of one
// group for larger D), and the group partials are summed through LDS.
constexpr int MERGE_THREADS = 256;
constexpr int MERGE_SPT = 16;  // splits per thread of the one-round-trip merge

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < MERGE_THREADS / 64; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(MERGE_THREADS) void attn_merge_kernel(AttnParams p) {
  __shared__ float red[MERGE_THREADS / 64];
  __shared__ float part[MERGE_THREADS];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / p.Hq;
  const int qh = bh - b * p.Hq;
  const int64_t base = (int64_t)bh * p.nsplit;
  const int ns = p.nsplit;
  const int D = p.D;
  const int dw = min(D, MERGE_THREADS);  // dims per pass
  const int groups = MERGE_THREADS / dw;  // split groups
  const int g = tid / dw;
  const int d0 = tid - g * dw;
  const int64_t obase = b * p.out.s[0] + qh * p.out.s[1];
  if (D <= MERGE_THREADS && ns <= groups * MERGE_SPT && ns <= MERGE_THREADS) {
    // One memory round trip: every load this thread needs (its acc partials of dim d0 over the
    // splits g, g + groups, ..., their m, and one (m, l) pair for the block reductions) goes out
    // before the first use; addresses are clamped to valid splits and the extra values masked.
    // The same sums in the same order as the loop form below, so the results are identical. In
    // the kernel trace the merge took 4.16 against 4.36 us (median over batch 1 and 8, 5-32
    // splits): most of a merge launch is the launch itself.
    float pa[MERGE_SPT], pm[MERGE_SPT];
    const int gc = min(g, groups - 1);
#pragma unroll
    for (int i = 0; i < MERGE_SPT; ++i) {
      const int sc = min(gc + i * groups, ns - 1);
      pa[i] = p.ws_acc[(base + sc) * D + d0];
      pm[i] = p.ws_m[base + sc];
    }
    const int tc = min(tid, ns - 1);
    const float mt0 = p.ws_m[base + tc];
    const float lt0 = p.ws_l[base + tc];
    const float mt = tid < ns ? mt0 : -INFINITY;
    const float M = block_reduce(mt, true, red);
    const float L =
        block_reduce((mt == -INFINITY) ? 0.0f : exp2f(mt - M) * lt0, false, red);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < MERGE_SPT; ++i) {
      const int s = g + i * groups;
      if (g < groups && s < ns) {
        const float w = (pm[i] == -INFINITY) ? 0.0f : exp2f(pm[i] - M);
        acc += w * pa[i];
      }
    }
    if (groups > 1) {
      part[tid] = acc;
      __syncthreads();
      if (g == 0) {
        for (int i = 1; i < groups; ++i) acc += part[i * dw + d0];
      }
    }
    if (g == 0) store_float(p.out.data, p.out.dtype, obase + d0 * p.out.s[2], acc / L);
    return;
  }
  float M = -INFINITY;
  for (int s = tid; s < ns; s += MERGE_THREADS) M = fmaxf(M, p.ws_m[base + s]);
  M = block_reduce(M, true, red);
  float L = 0.0f;
  for (int s = tid; s < ns; s += MERGE_THREADS) {
    const float ms = p.ws_m[base + s];
    L += (ms == -INFINITY) ? 0.0f : exp2f(ms - M) * p.ws_l[base + s];
  }
  L = block_reduce(L, false, red);

  for (int d = d0; d < D; d += dw) {
    float acc = 0.0f;
    if (g < groups) {
      // unrolled so that eight splits' loads are in flight before the first is used (one load
      // at a time left the merge latency-bound: 10.4 us at 64 splits, batch 1, ctx 16384)
#pragma unroll 8
      for (int s = g; s < ns; s += groups) {
        const float ms = p.ws_m[base + s];
        const float w = (ms == -INFINITY) ? 0.0f : exp2f(ms - M);
        acc += w * p.ws_acc[(base + s) * D + d];
      }
    }
    if (groups > 1) {
      part[tid] = acc;
      __syncthreads();
      if (g == 0) {
        for (int i = 1; i < groups; ++i) acc += part[i * dw + d0];
      }
      __syncthreads();
    }
    if (g == 0) store_float(p.out.data, p.out.dtype, obase + d * p.out.s[2], acc / L);
  }
}

// Split plan of the generic kernel: about 2048 waves in flight, at least 64 keys per split.
static SplitPlan plan_generic(int64_t B, int64_t Hq, int64_t S) {
  SplitPlan sp{};
  const int64_t rows = std::max<int64_t>(1, B * Hq);
  int64_t want = (2048 + rows - 1) / rows;
  const int64_t max_split = std::max<int64_t>(1, (S + 63) / 64);
  want = std::min(std::max<int64_t>(want, 1), max_split);
  int64_t chunk = (S + want - 1) / want;
  chunk = ((chunk + 63) / 64) * 64;
  sp.chunk = std::max<int64_t>(chunk, 64);
  sp.nsplit = (int)std::max<int64_t>(1, (S + sp.chunk - 1) / sp.chunk);
  return sp;
}

static size_t partial_bytes(int64_t B, int64_t Hq, int64_t D, int nsplit) {
  if (nsplit <= 1) return 0;
  const size_t slots = (size_t)(B * Hq) * (size_t)nsplit;
  // the arrival counters, then the m and l arrays, then acc; each rounded up to 256 bytes
  const size_t ml = ((slots * 4 + 255) / 256) * 256;
  return ARRIVAL_BYTES + 2 * ml + slots * (size_t)D * 4;
}

static void carve_workspace(AttnParams& p, void* ws) {
  const size_t slots = (size_t)(p.B * p.Hq) * (size_t)p.nsplit;
  const size_t ml = ((slots * 4 + 255) / 256) * 256;
  char* base = (char*)ws;
  p.ws_cnt = (uint32_t*)base;
  p.ws_m = (float*)(base + ARRIVAL_BYTES);
  p.ws_l = (float*)(base + ARRIVAL_BYTES + ml);
  p.ws_acc = (float*)(base + ARRIVAL_BYTES + 2 * ml);
}

// Split-K partials of lq_int4_decode_attention_noalloc: a static buffer on every device the
// library runs on, held until the process ends. 8 MiB: at 32 q / 8 KV heads, head_dim 128 any
// batch and context needs at most 2.0 MiB; larger needs (16 q heads per KV head, or head_dim
// 512, at some batch sizes) are rejected. In host code `scratch` names a host-side stand-in,
// never the device memory: the device address comes from hipGetSymbolAddress, once per device
// (scratch_address).
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)LQ_DECODE_ATTENTION_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::atomic<void*> scratch_ptr[MAX_DEVICES];
static std::mutex scratch_mutex;

// Device address of `scratch` on the device that runs `stream` (the current device for the
// legacy NULL stream), looked up on the first call for that device with the device made current.
static int scratch_address(hipStream_t stream, void** out) {
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return fail(LQ_ERR_HIP, "hipGetDevice failed");
  int dev = cur;
  if (stream != nullptr && hipStreamGetDevice(stream, &dev) != hipSuccess) {
    return fail(LQ_ERR_HIP, "hipStreamGetDevice failed");
  }
  if (dev < 0 || dev >= MAX_DEVICES) return fail(LQ_ERR_HIP, "device %d out of range", dev);
  void* ptr = scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(scratch_mutex);
    ptr = scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      if (dev != cur && hipSetDevice(dev) != hipSuccess) {
        return fail(LQ_ERR_HIP, "hipSetDevice(%d) failed", dev);
      }
      const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (dev != cur) (void)hipSetDevice(cur);
      if (e != hipSuccess || ptr == nullptr) {
        return fail(LQ_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
      }
      scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return LQ_OK;
}

// Where the split-K partials go: the caller's workspace, or the static per-device scratch.
struct PartialsBuffer {
  void* workspace;
  size_t workspace_bytes;
  bool use_scratch;
};

// The new token's K and V rows for lq_int4_decode_attention_pack (NULL: attention only).
struct NewToken {
  const lq_tensor* k;
  const lq_tensor* v;
};

static int decode_attention(const lq_tensor* q, const lq_tensor* k_packed,
                            const lq_tensor* v_packed, const lq_tensor* k_scale,
                            const lq_tensor* v_scale, const lq_tensor* mask, const lq_tensor* out,
                            int64_t seq_len, int num_key_value_groups, int group_size,
                            PartialsBuffer buf, void* stream, NewToken tok = {nullptr, nullptr});

}  // namespace lq

using namespace lq;

extern "C" size_t lq_int4_decode_attention_workspace(int64_t batch, int64_t n_q_heads,
                                                     int64_t n_kv_heads, int64_t head_dim,
                                                     int64_t seq_len, int group_size) {
  if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || seq_len <= 0) return 0;
  const SplitPlan g = plan_generic(batch, n_q_heads, seq_len);
  size_t need = partial_bytes(batch, n_q_heads, head_dim, g.nsplit);
  if (fast_path_shape_ok(head_dim, group_size, n_q_heads, n_kv_heads)) {
    const SplitPlan f = plan_fast(batch, n_kv_heads, seq_len);
    need = std::max(need, partial_bytes(batch, n_q_heads, head_dim, f.nsplit));
  }
  return need;
}

extern "C" int lq_int4_decode_attention(const lq_tensor* q, const lq_tensor* k_packed,
                                        const lq_tensor* v_packed, const lq_tensor* k_scale,
                                        const lq_tensor* v_scale, const lq_tensor* mask,
                                        const lq_tensor* out, int64_t seq_len,
                                        int num_key_value_groups, int group_size,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  return decode_attention(q, k_packed, v_packed, k_scale, v_scale, mask, out, seq_len,
                          num_key_value_groups, group_size,
                          PartialsBuffer{workspace, workspace_bytes, false}, stream);
}

extern "C" int lq_int4_decode_attention_pack(const lq_tensor* q, const lq_tensor* k_new,
                                             const lq_tensor* v_new, const lq_tensor* k_packed,
                                             const lq_tensor* v_packed, const lq_tensor* k_scale,
                                             const lq_tensor* v_scale, const lq_tensor* mask,
                                             const lq_tensor* out, int64_t seq_len,
                                             int num_key_value_groups, int group_size,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream) {
  if (k_new == nullptr || v_new == nullptr) {
    return fail(LQ_ERR_INVALID_ARG, "k_new and v_new are required");
  }
  return decode_attention(q, k_packed, v_packed, k_scale, v_scale, mask, out, seq_len,
                          num_key_value_groups, group_size,
                          PartialsBuffer{workspace, workspace_bytes, false}, stream,
                          NewToken{k_new, v_new});
}

extern "C" int lq_int4_decode_attention_noalloc(const lq_tensor* q, const lq_tensor* k_packed,
                                                const lq_tensor* v_packed,
                                                const lq_tensor* k_scale,
                                                const lq_tensor* v_scale, const lq_tensor* mask,
                                                const lq_tensor* out, int64_t seq_len,
                                                int num_key_value_groups, int group_size,
                                                void* stream) {
  return decode_attention(q, k_packed, v_packed, k_scale, v_scale, mask, out, seq_len,
                          num_key_value_groups, group_size, PartialsBuffer{nullptr, 0, true},
                          stream);
}

namespace lq {

static int decode_attention(const lq_tensor* q, const lq_tensor* k_packed,
                            const lq_tensor* v_packed, const lq_tensor* k_scale,
                            const lq_tensor* v_scale, const lq_tensor* mask, const lq_tensor* out,
                            int64_t seq_len, int num_key_value_groups, int group_size,
                            PartialsBuffer buf, void* stream, NewToken tok) {
  int rc;
  if (q == nullptr) return fail(LQ_ERR_INVALID_ARG, "q: descriptor is NULL");
  const int qdim = q->ndim;
  if (qdim != 3 && qdim != 4) {
    return fail(LQ_ERR_INVALID_ARG, "q: expected [B, Hq, 1, D] or [B, Hq, D], got %d dims", qdim);
  }
  if ((rc = check_tensor(q, "q", qdim, true)) != LQ_OK) return rc;
  if (qdim == 4 && q->shape[2] != 1) {
    return fail(LQ_ERR_INVALID_ARG, "Fused INT4 decode attention expects q_len=1, got %lld",
                (long long)q->shape[2]);
  }
  if ((rc = check_tensor(k_packed, "k_packed", 4, false, LQ_U8)) != LQ_OK) return rc;
  if ((rc = check_tensor(v_packed, "v_packed", 4, false, LQ_U8)) != LQ_OK) return rc;
  if ((rc = check_tensor(k_scale, "k_scale", 4, false, LQ_F32)) != LQ_OK) return rc;
  if ((rc = check_tensor(v_scale, "v_scale", 4, false, LQ_F32)) != LQ_OK) return rc;
  if ((rc = check_tensor(out, "out", 3, true)) != LQ_OK) return rc;
  const int64_t B = q->shape[0], Hq = q->shape[1], D = q->shape[qdim - 1];
  const int64_t Hkv = k_packed->shape[1], cap = k_packed->shape[2];
  if (group_size <= 0 || group_size % 2 != 0 || D % group_size != 0) {
    return fail(LQ_ERR_INVALID_ARG, "head_dim=%lld must be divisible by an even group_size=%d",
                (long long)D, group_size);
  }
  if (D > GEN_MAX_D || D % 2 != 0) {
    return fail(LQ_ERR_UNSUPPORTED, "head_dim=%lld unsupported (even, <= %d)", (long long)D,
                GEN_MAX_D);
  }
  if (num_key_value_groups <= 0 || Hkv * num_key_value_groups != Hq) {
    return fail(LQ_ERR_INVALID_ARG, "n_q_heads=%lld != n_kv_heads=%lld * groups=%d",
                (long long)Hq, (long long)Hkv, num_key_value_groups);
  }
  const lq_tensor* caches[2] = {k_packed, v_packed};
  for (const lq_tensor* c : caches) {
    if (c->shape[0] != B || c->shape[1] != Hkv || c->shape[2] != cap || c->shape[3] != D / 2) {
      return fail(LQ_ERR_INVALID_ARG, "packed caches must be [%lld, %lld, %lld, %lld]",
                  (long long)B, (long long)Hkv, (long long)cap, (long long)(D / 2));
    }
  }
  const lq_tensor* scales[2] = {k_scale, v_scale};
  for (const lq_tensor* s : scales) {
    if (s->shape[0] != B || s->shape[1] != Hkv || s->shape[2] != cap ||
        s->shape[3] != D / group_size) {
      return fail(LQ_ERR_INVALID_ARG, "scale caches must be [%lld, %lld, %lld, %lld]",
                  (long long)B, (long long)Hkv, (long long)cap, (long long)(D / group_size));
    }
  }
  if (out->shape[0] != B || out->shape[1] != Hq || out->shape[2] != D) {
    return fail(LQ_ERR_INVALID_ARG, "out must be [%lld, %lld, %lld]", (long long)B, (long long)Hq,
                (long long)D);
  }
  if (seq_len < 1 || seq_len > cap) {
    return fail(LQ_ERR_INVALID_ARG, "seq_len=%lld outside [1, capacity=%lld]",
                (long long)seq_len, (long long)cap);
  }
  if (mask != nullptr) {
    if ((rc = check_tensor(mask, "mask", 4, false, LQ_F32)) != LQ_OK) return rc;
    if (mask->shape[0] != B) {
      return fail(LQ_ERR_INVALID_ARG, "mask batch %lld != %lld", (long long)mask->shape[0],
                  (long long)B);
    }
  }
  if (tok.k != nullptr) {
    // the token tensors as lq_int4_pack_kv_pair checks them, one token into row seq_len - 1
    if ((rc = pack_pair_at(tok.k, tok.v, k_packed, v_packed, k_scale, v_scale, seq_len - 1,
                           group_size, false, nullptr, "")) != LQ_OK) {
      return rc;
    }
    if (tok.k->shape[2] != 1 || tok.v->shape[2] != 1) {
      return fail(LQ_ERR_INVALID_ARG, "k_new and v_new must hold one token ([B, Hkv, 1, D])");
    }
  }
  if (B == 0 || Hq == 0) return LQ_OK;

  AttnParams p{};
  p.q.data = q->data;
  p.q.dtype = q->dtype;
  p.q.s[0] = q->stride[0];
  p.q.s[1] = q->stride[1];
  p.q.s[2] = q->stride[qdim - 1];
  p.kp = (const uint8_t*)k_packed->data;
  p.vp = (const uint8_t*)v_packed->data;
  p.ks = (const float*)k_scale->data;
  p.vs = (const float*)v_scale->data;
  for (int i = 0; i < 4; ++i) {
    p.kps[i] = k_packed->stride[i];
    p.vps[i] = v_packed->stride[i];
    p.kss[i] = k_scale->stride[i];
    p.vss[i] = v_scale->stride[i];
  }
  if (mask != nullptr) {
    p.mask = (const float*)mask->data;
    p.mask_sb = mask->stride[0];
    p.mask_sk = mask->stride[3];
    p.mask_len = mask->shape[3];
  }
  p.out = make_view(out);
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.D = (int)D;
  p.g = group_size;
  p.nrep = num_key_value_groups;
  p.S = seq_len;
  p.scale_sm = (float)(1.4426950408889634 / sqrt((double)D));

  const bool fast = fast_path_ok(p);
  if (!fast && diag(LQ_DIAG_ATTN_REQUIRE_FAST)) {  // tests: the call must take the MFMA kernel
    return fail(LQ_ERR_INVALID_ARG,
                "LQ_ATTN_REQUIRE_FAST is set and this call takes the generic kernel");
  }
  if (tok.k != nullptr && fast) {  // the MFMA kernel packs the token itself
    auto row_view = [](const lq_tensor* t) {
      View v{t->data, t->dtype, {t->stride[0], t->stride[1], t->stride[3], 0}};
      return v;
    };
    p.knew = row_view(tok.k);
    p.vnew = row_view(tok.v);
    p.pack = 1;
  }
  const SplitPlan sp = fast ? plan_fast(B, Hkv, seq_len) : plan_generic(B, Hq, seq_len);
  p.nsplit = sp.nsplit;
  p.chunk = sp.chunk;
  const size_t need = partial_bytes(B, Hq, D, p.nsplit);
  hipStream_t st = (hipStream_t)stream;
  if (need > 0 && buf.use_scratch) {
    if (need > NOALLOC_SCRATCH_BYTES) {
      return fail(LQ_ERR_WORKSPACE,
                  "lq_int4_decode_attention_noalloc: this shape needs %zu bytes of split-K "
                  "partials, more than the library's %zu-byte static scratch; call "
                  "lq_int4_decode_attention with a workspace instead", need,
                  NOALLOC_SCRATCH_BYTES);
    }
    void* ptr = nullptr;
    if ((rc = scratch_address(st, &ptr)) != LQ_OK) return rc;
    carve_workspace(p, ptr);
  } else if (need > 0) {
    if (buf.workspace == nullptr || buf.workspace_bytes < need) {
      return fail(LQ_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                  buf.workspace == nullptr ? (size_t)0 : buf.workspace_bytes);
    }
    if (((uintptr_t)buf.workspace & 255) != 0) {
      return fail(LQ_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    }
    carve_workspace(p, buf.workspace);
  }

  if (tok.k != nullptr && !fast) {  // the generic kernel reads row seq_len - 1: pack it first
    if ((rc = pack_pair_at(tok.k, tok.v, k_packed, v_packed, k_scale, v_scale, seq_len - 1,
                           group_size, true, st, "lq_int4_decode_attention_pack (pack)")) != LQ_OK) {
      return rc;
    }
  }
  // on request, the MFMA kernel merges its own splits when the unit count fits the counters
  p.fold = fast && p.nsplit > 1 && B * Hkv <= ARRIVAL_UNITS &&
           fast_fold_fits(num_key_value_groups, p.nsplit) && diag(LQ_DIAG_ATTN_FOLD_MERGE);
  if (fast) {
    if ((rc = launch_fast(p, st)) != LQ_OK) return rc;
  } else {
    hipLaunchKernelGGL(attn_generic_kernel, dim3((unsigned)(B * Hq), (unsigned)p.nsplit),
                       dim3(64), 0, st, p);
    if ((rc = check_launch("lq_int4_decode_attention")) != LQ_OK) return rc;
  }
  if (p.nsplit > 1 && !p.fold) {
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(B * Hq)), dim3(MERGE_THREADS), 0, st, p);
    if ((rc = check_launch("lq_int4_decode_attention merge")) != LQ_OK) return rc;
  }
  return LQ_OK;
}

}  // namespace lq
