// INT4 prefill attention: causal multi-token attention of q [B, Hq, L, D] over the packed cache,
// query position t of head h reading keys 0 .. t of KV head h / n_rep, the semantics of the
// reference's _int4_prefill_attention_kernel (hybrid_quant/int4_8b_attention.py:114-251, launched
// by _prefill_attention at :594-625; scores (q . k) * log2(e)/sqrt(D), exp2-domain softmax).
//
//   * prefill_mfma_kernel: head_dim 128, group 32/64/128, bf16 queries, contiguous key rows.
//   * prefill_generic_kernel: any even group dividing any head_dim <= 512, any query dtype; one
//     wave per (batch, head, position), fp32 VALU throughout.
//
// MFMA path. A workgroup of 4 waves shares one (batch, KV head) and walks its keys in tiles of
// 32; each wave owns 32 query positions of one query head (the 4 waves are the n_rep heads of one
// position block, or several position blocks when n_rep < 4). Per tile the workgroup loads the
// packed K and V rows and their scales once, decodes the nibbles once into LDS as bf16 operands,
// and every wave reads them from there:
//   K tile  [key][dim]  in MFMA A-operand order (8-dim octets in slot order 0,4,1,5,2,6,3,7);
//   V tile  [dim][key]  transposed, keys permuted so a lane group's 8 keys are contiguous;
//   scales  [group][key] (log2(e)/sqrt(D) folded into the key scales).
// Nibbles decode to exact fp16 integers: bits 0x6400 | (n ^ 8) are the value 1032 + n, and one
// packed fp16 add per pair subtracts 1032.
//
// Products use v_mfma_f32_16x16x32_f16 (D[16x16] += A[16x32] * B[32x16]; lane l holds A row
// l%16 and B column l%16 with K slots 8*(l/16) .. +7, and D rows 4*(l/16) .. +3 of column l%16).
//   S^T[key][query] per group m: A = K rows (exact integers), B = Q^T scaled by a power of two
//     2^-e per query row so that its largest value lies in [2^14, 2^15) (bf16 queries are then
//     exact in fp16, products exact, sums fp32); the group partials are scaled by the fp32 key
//     scale of group m and summed in fp32, as the reference sums nibble * scale * q in fp32, and
//     2^e multiplies the score inside the softmax's exp2 argument.
//   O^T[dim][query]: A = V^T rows (exact integers) of the dims of group m, B = P'_m with
//     P'_m[key][query] = p[key][query] * vscale[key][m] / vmax_m split into fp16 hi + lo (two
//     MFMAs, about 22 significant bits; hi the fp16 product of p and the scale rounded to fp16,
//     lo the fp32 remainder rounded to fp16), vmax_m the power of two at or above the largest V scale of group m over the
//     workgroup's keys (one pre-pass over the scales), so P'_m <= 2^8 never overflows fp16; the
//     output tiles of group m are multiplied by vmax_m at the end.
// Softmax runs in the exp2 domain with a lazily moved running max (rescale only when a score
// exceeds it by more than 8, so p <= 2^8), as in the decode kernel.
#include <math.h>
#include <stdlib.h>

#include "lq_common.h"

namespace lq {
namespace {

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int PD = 128;      // head_dim of the MFMA path
constexpr int KT = 32;       // keys per tile
constexpr int QW = 32;       // query positions per wave (two 16-column tiles)
constexpr int NW = 4;        // waves per workgroup
constexpr int KROW = PD + 8; // bf16 per key row of the K tile (272 B: rows 4 banks apart)
constexpr int VROW = KT + 8; // bf16 per dim row of the V^T tile (80 B)
constexpr float LAZY = 8.0f; // running-max slack of the lazy rescale (p <= 2^LAZY)
constexpr int PG_MAX_D = 512;

struct PrefillParams {
  View q;    // strides of (b, h, t, d)
  View out;  // strides of (b, h, t, d)
  const uint8_t* kp;
  const uint8_t* vp;
  int64_t kps[4], vps[4];
  const float* ks;
  const float* vs;
  int64_t kss[4], vss[4];
  int B, Hq, Hkv, D, g, nrep, L;
  float scale_sm;  // log2(e) / sqrt(D)
};

__device__ __forceinline__ f32x4_t mfma_f16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// exact fp16 pair n from the nibbles at bits 3:0 and 19:16 of x: 1032 + n, minus 1032
__device__ __forceinline__ uint32_t nib_pair_f16(uint32_t x) {
  const uint32_t m = ((x ^ 0x00080008u) & 0x000F000Fu) | 0x64006400u;
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, m) +
                                          __builtin_bit_cast(f16x2_t, 0xE408E408u));
}

// 8 nibbles of one dword -> fp16 n in slot order of dims (0, 4, 1, 5, 2, 6, 3, 7)
__device__ __forceinline__ u32x4_t decode_octet_f16(uint32_t w) {
  u32x4_t o;
  o.x = nib_pair_f16(w);
  o.y = nib_pair_f16(w >> 4);
  o.z = nib_pair_f16(w >> 8);
  o.w = nib_pair_f16(w >> 12);
  return o;
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

template <int G>
struct alignas(16) PrefillLds {
  uint16_t k[2][KT][KROW];
  uint16_t v[2][PD][VROW];
  float ks[2][G][KT];
  float vs[2][G][KT];
  uint16_t vp[2][G][KT];  // vs as fp16, in the P V B-operand order (vpair_slot)
  float vred[NW][G];
};

// One thread's share of a tile's global reads: 8 bytes of K (key tid/8, dwords 2u, 2u+1),
// dword tid/16 of the V rows of keys 2(tid%16), 2(tid%16)+1 (consecutive lanes take consecutive
// key pairs, so the transposed LDS writes of a wave fill whole rows instead of hitting one bank
// per row 8 apart), and one scale word (K scales on threads 0..127, V scales on 128..255). Keys
// at or past L read as zero.
struct RawTile {
  uint32_t k0, k1;
  uint32_t v0, v1;
  float sc;
};

template <int G>
__device__ __forceinline__ void load_tile(const uint8_t* kb, const uint8_t* vb, const float* ksb,
                                          const float* vsb, int L, int tb, int tid, RawTile& r) {
  const int kk = tb + (tid >> 3);
  if (kk < L) {
    const uint2 w = *(const uint2*)(kb + (int64_t)kk * 64 + 8 * (tid & 7));
    r.k0 = w.x;
    r.k1 = w.y;
  } else {
    r.k0 = 0;
    r.k1 = 0;
  }
  const int vk = tb + 2 * (tid & 15);
  r.v0 = vk < L ? *(const uint32_t*)(vb + (int64_t)vk * 64 + 4 * (tid >> 4)) : 0u;
  r.v1 = vk + 1 < L ? *(const uint32_t*)(vb + (int64_t)(vk + 1) * 64 + 4 * (tid >> 4)) : 0u;
  const int si = tid & 127;
  const int sk = tb + (si & (KT - 1));  // scale word (key si % 32, group si / 32)
  const float* sb = tid < 128 ? ksb : vsb;
  r.sc = (si < G * KT && sk < L) ? sb[(int64_t)sk * G + (si / KT)] : 0.0f;
}

// key k of a tile -> its half-word in the fp16 V-scale row: lane group j's B-operand key pairs
// (16t + 4j + r, r + 1), t = u >> 1, r = 2 (u & 1), are dword 4j + u, so a lane reads its four
// pairs with one 16-byte load
__device__ __forceinline__ int vpair_slot(int k) { return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3); }

// key k of a tile -> its column in the V^T tile: lane group j's keys 4j..4j+3 and 16+4j..16+4j+3
// (its K slots 0..7 of the P V product) sit at columns 8j .. 8j+7
__device__ __forceinline__ int vcol(int k) { return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3); }

template <int G>
__device__ __forceinline__ void stage_tile(PrefillLds<G>& s, int nb, const RawTile& r, int tid,
                                           float scale_sm, const float (&vinv)[G]) {
  {
    const int key = tid >> 3;
    const int u = tid & 7;
    *(u32x4_t*)&s.k[nb][key][16 * u] = decode_octet_f16(r.k0);
    *(u32x4_t*)&s.k[nb][key][16 * u + 8] = decode_octet_f16(r.k1);
  }
  {
    const int k0 = 2 * (tid & 15);
    const int w = tid >> 4;
    const int col = vcol(k0);
    // ylo = bytes (k0.b0, k0.b1, k1.b0, k1.b1), yhi = (k0.b2, k0.b3, k1.b2, k1.b3): nibble i of
    // ylo and of ylo >> 16 is dim 8w + i of key k0 and of key k0 + 1
    const uint32_t ylo = __builtin_amdgcn_perm(r.v1, r.v0, 0x05040100u);
    const uint32_t yhi = __builtin_amdgcn_perm(r.v1, r.v0, 0x07060302u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *(uint32_t*)&s.v[nb][8 * w + i][col] = nib_pair_f16(ylo >> (4 * i));
      *(uint32_t*)&s.v[nb][8 * w + 4 + i][col] = nib_pair_f16(yhi >> (4 * i));
    }
  }
  const int si = tid & 127;
  if (si < G * KT) {  // consecutive lanes write consecutive keys of one group (no bank conflict)
    const int key = si & (KT - 1);
    const int m = si / KT;
    if (tid < 128) {
      s.ks[nb][m][key] = r.sc * scale_sm;
    } else {
      const float v = r.sc * vinv[m];
      s.vs[nb][m][key] = v;
      s.vp[nb][m][vpair_slot(key)] = __builtin_bit_cast(uint16_t, (_Float16)v);
    }
  }
}

template <int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_mfma_kernel(PrefillParams p) {
  constexpr int CPG = 4 / G;  // 32-dim chunks per group
  constexpr int NT = 8 / G;   // 16-dim output tiles per group
  __shared__ PrefillLds<G> lds;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j4 = lane >> 4;
  const int c16 = lane & 15;
  const int L = p.L;
  const int unit = blockIdx.y;  // (batch, KV head)
  const int b = unit / p.Hkv;
  const int kvh = unit - b * p.Hkv;

  // rows (position block, head of the group), position-block major; heavy blocks launch first
  const int npb = (L + QW - 1) / QW;
  const int rows = npb * p.nrep;
  const int wg = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int row = wg * NW + wave;
  const bool active = row < rows;
  const int pb = active ? row / p.nrep : 0;
  const int head = kvh * p.nrep + (active ? row - pb * p.nrep : 0);
  const int q0 = pb * QW;
  const int wend = min(L, q0 + QW);  // this wave reads keys [0, wend)
  const int last_row = min(wg * NW + NW - 1, rows - 1);
  const int gend = min(L, (last_row / p.nrep) * QW + QW);  // the workgroup's key range
  const int nsteps = (gend + KT - 1) / KT;

  const uint8_t* kb = p.kp + b * p.kps[0] + kvh * p.kps[1];
  const uint8_t* vb = p.vp + b * p.vps[0] + kvh * p.vps[1];
  const float* ksb = p.ks + b * p.kss[0] + kvh * p.kss[1];
  const float* vsb = p.vs + b * p.vss[0] + kvh * p.vss[1];

  RawTile raw;
  load_tile<G>(kb, vb, ksb, vsb, L, 0, tid, raw);

  // vmax_m: power of two at or above the largest V scale of group m over keys [0, gend)
  float vpow[G], vinv[G];
  {
    float mx[G];
#pragma unroll
    for (int m = 0; m < G; ++m) mx[m] = 0.0f;
    // eight keys' scales in flight per thread: one key per iteration waited out a full memory
    // round trip each time (64 of them for a workgroup at the end of a 16K-token prompt)
    constexpr int PRE = 8;
    int k = tid;
    for (; k + (PRE - 1) * 256 < gend; k += PRE * 256) {
      float v[PRE][G];
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
#pragma unroll
        for (int m = 0; m < G; ++m) v[u][m] = vsb[(int64_t)(k + u * 256) * G + m];
      }
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
#pragma unroll
        for (int m = 0; m < G; ++m) mx[m] = fmaxf(mx[m], v[u][m]);
      }
    }
    for (; k < gend; k += 256) {
#pragma unroll
      for (int m = 0; m < G; ++m) mx[m] = fmaxf(mx[m], vsb[(int64_t)k * G + m]);
    }
#pragma unroll
    for (int m = 0; m < G; ++m) {
      const float w = group_max<64>(mx[m]);
      if (lane == 0) lds.vred[wave][m] = w;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < G; ++m) {
      float v = lds.vred[0][m];
#pragma unroll
      for (int w = 1; w < NW; ++w) v = fmaxf(v, lds.vred[w][m]);
      const uint32_t bits = __float_as_uint(v);
      const int e = (int)((bits >> 23) & 0xffu) - 127 + ((bits & 0x7fffffu) != 0 ? 1 : 0);
      const bool ok = v > 0.0f && e > -120 && e < 120;  // normal, finite scales
      vpow[m] = ok ? __uint_as_float((uint32_t)(127 + e) << 23) : 1.0f;
      vinv[m] = ok ? __uint_as_float((uint32_t)(127 - e) << 23) : 1.0f;
    }
  }
  stage_tile<G>(lds, 0, raw, tid, p.scale_sm, vinv);
  if (nsteps > 1) load_tile<G>(kb, vb, ksb, vsb, L, KT, tid, raw);

  // Query operands: lane (j4, c16) of column tile qt holds position q0 + 16 qt + c16, dims
  // 32c + 8 j4 + (0,4,1,5,2,6,3,7) for chunk c, as fp16 q * 2^-e with 2^e (qsc) chosen per row
  // so that max |q| * 2^-e lies in [2^14, 2^15).
  u32x4_t qop[2][4];
  float qsc[2];
  {
    const uint16_t* qbits = (const uint16_t*)p.q.data;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int pos = q0 + 16 * qt + c16;
      const bool ok = active && pos < L;
      // every lane loads from a valid row (position clamped to L - 1) and masks afterwards: a load
      // under `ok` became a branch with its own wait, 64 round trips in a row per wave
      const int64_t base =
          b * p.q.s[0] + (int64_t)head * p.q.s[1] + (int64_t)min(pos, L - 1) * p.q.s[2];
      float qv[4][8];
      float mx = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float x = bf16_bits_to_float(qbits[base + (32 * c + 8 * j4 + u) * p.q.s[3]]);
          qv[c][u] = ok ? x : 0.0f;
          mx = fmaxf(mx, fabsf(qv[c][u]));
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      int e = mx > 0.0f ? (int)((__float_as_uint(mx) >> 23) & 0xffu) - 127 - 14 : 0;
      e = max(-100, min(100, e));
      qsc[qt] = __uint_as_float((uint32_t)(127 + e) << 23);
      const float qinv = __uint_as_float((uint32_t)(127 - e) << 23);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int u = 0; u < 4; ++u) qop[qt][c][u] = pack_f16(qv[c][u] * qinv, qv[c][u + 4] * qinv);
      }
    }
  }

  f32x4_t o[2][8];
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.0f, 0.0f};
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[qt][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }

  for (int st = 0; st < nsteps; ++st) {
    __syncthreads();  // tile st is staged; the other buffer is free
    if (st + 1 < nsteps) {
      stage_tile<G>(lds, (st + 1) & 1, raw, tid, p.scale_sm, vinv);
      if (st + 2 < nsteps) load_tile<G>(kb, vb, ksb, vsb, L, (st + 2) * KT, tid, raw);
    }
    const int tb = st * KT;
    if (!active || tb >= wend) continue;
    const int nb = st & 1;

    // ---- scores S^T[key][query]: lane holds keys tb + 16t + 4 j4 + r of query column c16
    u32x4_t ka[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int c = 0; c < 4; ++c) ka[t][c] = *(const u32x4_t*)&lds.k[nb][16 * t + c16][32 * c + 8 * j4];
    }
    f32x4_t s[2][2];
#pragma unroll
    for (int m = 0; m < G; ++m) {
      f32x4_t ks4[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) ks4[t] = *(const f32x4_t*)&lds.ks[nb][m][16 * t + 4 * j4];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int cc = 0; cc < CPG; ++cc) acc = mfma_f16(ka[t][m * CPG + cc], qop[qt][m * CPG + cc], acc);
          s[qt][t] = (m == 0) ? acc * ks4[t] : s[qt][t] + acc * ks4[t];
        }
      }
    }
    if (tb == q0) {  // diagonal tile: keys after the query position are masked
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (16 * t + 4 * j4 + r > 16 * qt + c16) s[qt][t][r] = -INFINITY;
          }
        }
      }
    }

    // ---- softmax (lazy running max), then per group m: P'_m and the P V products
    float pr[2][2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float lm = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) lm = fmaxf(lm, s[qt][t][r]);
      }
      lm *= qsc[qt];  // scores are s * 2^e
      if (__any(lm > m_run[qt] + LAZY)) {
        float mt = fmaxf(lm, __shfl_xor(lm, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run[qt], mt);
        // accumulators are still zero while m_run is -inf
        const float alpha =
            (m_run[qt] == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[qt] - m_new);
        if (alpha != 1.0f) {
#pragma unroll
          for (int i = 0; i < 8; ++i) o[qt][i] *= alpha;
          l_run[qt] *= alpha;
        }
        m_run[qt] = m_new;
      }
      float psum = 0.0f;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pr[qt][t][r] = __builtin_amdgcn_exp2f(fmaf(s[qt][t][r], qsc[qt], -m_run[qt]));
          psum += pr[qt][t][r];
        }
      }
      l_run[qt] += psum;
    }
    // Wave priority 1 over P' and the P V products: of the two waves on a SIMD, the one in this
    // section issues first, the other's QK and softmax work filling in behind it (L = 16384:
    // 4.47 against 4.89 ms; the same over the QK products gains nothing)
    __builtin_amdgcn_s_setprio(1);
    // B operand slots 2u, 2u+1 = keys (t, r) = (u >> 1, 2(u & 1)) and (u >> 1, 2(u & 1) + 1)
    uint32_t p16[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        p16[qt][u] = pack_f16(pr[qt][u >> 1][2 * (u & 1)], pr[qt][u >> 1][2 * (u & 1) + 1]);
      }
    }
#pragma unroll
    for (int m = 0; m < G; ++m) {
      f32x4_t vs4[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) vs4[t] = *(const f32x4_t*)&lds.vs[nb][m][16 * t + 4 * j4];
      const u32x4_t vs16 = *(const u32x4_t*)&lds.vp[nb][m][8 * j4];
      // P'_m = p * vs as fp16 hi + lo (about 22 significant bits): hi = RN(RN16(p) * RN16(vs))
      // by one packed fp16 multiply per pair, within 2^-10 of p * vs; lo = RN16(p * vs - hi)
      // with p * vs exact inside the fused multiply-add (four instructions per pair; rounding
      // p * vs itself to fp16 took two fp32 multiplies and a conversion for hi)
      u32x4_t bhi[2], blo[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int t = u >> 1;
          const int r = 2 * (u & 1);
          // (the element is copied out first: __builtin_bit_cast of an ext_vector element reads
          // element 0 whatever the index with this compiler)
          const uint32_t vw = vs16[u];
          const f16x2_t hh = __builtin_bit_cast(f16x2_t, p16[qt][u]) * __builtin_bit_cast(f16x2_t, vw);
          bhi[qt][u] = __builtin_bit_cast(uint32_t, hh);
          blo[qt][u] = pack_f16(__builtin_fmaf(pr[qt][t][r], vs4[t][r], -(float)hh[0]),
                                __builtin_fmaf(pr[qt][t][r + 1], vs4[t][r + 1], -(float)hh[1]));
        }
      }
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const int it = m * NT + i;
        const u32x4_t va = *(const u32x4_t*)&lds.v[nb][16 * it + c16][8 * j4];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[qt][it] = mfma_f16(va, bhi[qt], o[qt][it]);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[qt][it] = mfma_f16(va, blo[qt], o[qt][it]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  }

  if (!active) return;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float l = l_run[qt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = 1.0f / l;
    const int pos = q0 + 16 * qt + c16;
    if (pos >= L) continue;
    const int64_t obase = b * p.out.s[0] + (int64_t)head * p.out.s[1] + (int64_t)pos * p.out.s[2];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = o[qt][it][r] * (vpow[it / NT] * inv);
        store_float(p.out.data, p.out.dtype, obase + (int64_t)(16 * it + 4 * j4 + r) * p.out.s[3], v);
      }
    }
  }
}

// One wave per (batch, query head, position t): keys 0 .. t in blocks of 64, one key per lane for
// the scores, then the V rows of the block accumulated lane-per-dim.
__global__ __launch_bounds__(64) void prefill_generic_kernel(PrefillParams p) {
  __shared__ float q_s[PG_MAX_D];
  __shared__ float p_s[64];
  const int lane = threadIdx.x;
  const int t = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.Hq;
  const int qh = bh - b * p.Hq;
  const int kvh = qh / p.nrep;
  const int D = p.D;
  const int g = p.g;
  const int groups = D / g;
  const int64_t qoff = b * p.q.s[0] + (int64_t)qh * p.q.s[1] + (int64_t)t * p.q.s[2];
  for (int d = lane; d < D; d += 64) q_s[d] = load_float(p.q.data, p.q.dtype, qoff + d * p.q.s[3]);
  __syncthreads();

  const uint8_t* kbase = p.kp + b * p.kps[0] + kvh * p.kps[1];
  const uint8_t* vbase = p.vp + b * p.vps[0] + kvh * p.vps[1];
  const float* ksbase = p.ks + b * p.kss[0] + kvh * p.kss[1];
  const float* vsbase = p.vs + b * p.vss[0] + kvh * p.vss[1];
  float m = -INFINITY;
  float l = 0.0f;
  float acc[PG_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < PG_MAX_D / 64; ++i) acc[i] = 0.0f;

  const int64_t kend = (int64_t)t + 1;
  for (int64_t start = 0; start < kend; start += 64) {
    const int64_t n = start + lane;
    float s = -INFINITY;
    if (n < kend) {
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
    }
    const float m_new = fmaxf(m, group_max<64>(s));  // finite: key 0 is in the first block
    const float alpha = exp2f(m - m_new);
    const float pn = (s == -INFINITY) ? 0.0f : exp2f(s - m_new);
    l = l * alpha + group_sum<64>(pn);
    p_s[lane] = pn;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PG_MAX_D / 64; ++i) acc[i] *= alpha;
    const int cnt = (int)min((int64_t)64, kend - start);
    for (int jj = 0; jj < cnt; ++jj) {
      const float pj = p_s[jj];
      const uint8_t* vr = vbase + (start + jj) * p.vps[2];
      const float* vsr = vsbase + (start + jj) * p.vss[2];
#pragma unroll
      for (int i = 0; i < PG_MAX_D / 64; ++i) {
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
  const int64_t ooff = b * p.out.s[0] + (int64_t)qh * p.out.s[1] + (int64_t)t * p.out.s[2];
#pragma unroll
  for (int i = 0; i < PG_MAX_D / 64; ++i) {
    const int d = lane + 64 * i;
    if (d < D) store_float(p.out.data, p.out.dtype, ooff + d * p.out.s[3], acc[i] / l);
  }
}

bool prefill_mfma_ok(const PrefillParams& p) {
  if (diag(LQ_DIAG_PREFILL_FORCE_GENERIC)) return false;
  if (p.D != PD || (p.g != 32 && p.g != 64 && p.g != 128)) return false;
  if (p.q.dtype != LQ_BF16) return false;
  const int64_t G = PD / p.g;
  // contiguous key rows (64 packed bytes, G scale words); 8-byte K and 4-byte V/scale alignment
  if (p.kps[3] != 1 || p.vps[3] != 1 || p.kps[2] != 64 || p.vps[2] != 64) return false;
  if (p.kss[3] != 1 || p.vss[3] != 1 || p.kss[2] != G || p.vss[2] != G) return false;
  if (p.kps[0] % 8 != 0 || p.kps[1] % 8 != 0 || ((uintptr_t)p.kp & 7) != 0) return false;
  if (p.vps[0] % 4 != 0 || p.vps[1] % 4 != 0 || ((uintptr_t)p.vp & 3) != 0) return false;
  if (((uintptr_t)p.ks & 3) != 0 || ((uintptr_t)p.vs & 3) != 0) return false;
  return true;
}

template <int G>
void launch_mfma(const PrefillParams& p, hipStream_t st) {
  const int64_t npb = ((int64_t)p.L + QW - 1) / QW;
  const int64_t nwg = (npb * p.nrep + NW - 1) / NW;
  hipLaunchKernelGGL((prefill_mfma_kernel<G>), dim3((unsigned)nwg, (unsigned)(p.B * p.Hkv)),
                     dim3(256), 0, st, p);
}

}  // namespace
}  // namespace lq

using namespace lq;

extern "C" int lq_int4_prefill_attention(const lq_tensor* q, const lq_tensor* k_packed,
                                         const lq_tensor* v_packed, const lq_tensor* k_scale,
                                         const lq_tensor* v_scale, const lq_tensor* out,
                                         int num_key_value_groups, int group_size, void* stream) {
  int rc;
  if ((rc = check_tensor(q, "q", 4, true)) != LQ_OK) return rc;
  if ((rc = check_tensor(k_packed, "k_packed", 4, false, LQ_U8)) != LQ_OK) return rc;
  if ((rc = check_tensor(v_packed, "v_packed", 4, false, LQ_U8)) != LQ_OK) return rc;
  if ((rc = check_tensor(k_scale, "k_scale", 4, false, LQ_F32)) != LQ_OK) return rc;
  if ((rc = check_tensor(v_scale, "v_scale", 4, false, LQ_F32)) != LQ_OK) return rc;
  if ((rc = check_tensor(out, "out", 4, true)) != LQ_OK) return rc;
  const int64_t B = q->shape[0], Hq = q->shape[1], L = q->shape[2], D = q->shape[3];
  const int64_t Hkv = k_packed->shape[1], cap = k_packed->shape[2];
  if (group_size <= 0 || group_size % 2 != 0 || D % group_size != 0) {
    return fail(LQ_ERR_INVALID_ARG, "head_dim=%lld must be divisible by an even group_size=%d",
                (long long)D, group_size);
  }
  if (D > PG_MAX_D || D % 2 != 0) {
    return fail(LQ_ERR_UNSUPPORTED, "head_dim=%lld unsupported (even, <= %d)", (long long)D,
                PG_MAX_D);
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
  if (out->shape[0] != B || out->shape[1] != Hq || out->shape[2] != L || out->shape[3] != D) {
    return fail(LQ_ERR_INVALID_ARG, "out must be [%lld, %lld, %lld, %lld]", (long long)B,
                (long long)Hq, (long long)L, (long long)D);
  }
  if (L > cap) {
    return fail(LQ_ERR_INVALID_ARG, "q_len=%lld exceeds the cache capacity %lld", (long long)L,
                (long long)cap);
  }
  if (L >= ((int64_t)1 << 30) || B * Hq > 65535 || B * Hkv > 65535) {
    return fail(LQ_ERR_UNSUPPORTED, "prefill of B=%lld Hq=%lld L=%lld exceeds the launch limits",
                (long long)B, (long long)Hq, (long long)L);
  }
  if (B == 0 || Hq == 0 || L == 0) return LQ_OK;

  PrefillParams p{};
  p.q = make_view(q);
  p.out = make_view(out);
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
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.D = (int)D;
  p.g = group_size;
  p.nrep = num_key_value_groups;
  p.L = (int)L;
  p.scale_sm = (float)(1.4426950408889634 / sqrt((double)D));

  hipStream_t st = (hipStream_t)stream;
  const bool mfma = prefill_mfma_ok(p);
  if (!mfma && diag(LQ_DIAG_PREFILL_REQUIRE_MFMA)) {  // tests: the call must take the MFMA kernel
    return fail(LQ_ERR_INVALID_ARG,
                "LQ_PREFILL_REQUIRE_MFMA is set and this call takes the generic kernel");
  }
  if (mfma) {
    switch (PD / group_size) {
      case 4: launch_mfma<4>(p, st); break;
      case 2: launch_mfma<2>(p, st); break;
      default: launch_mfma<1>(p, st); break;
    }
    return check_launch("lq_int4_prefill_attention (mfma)");
  }
  hipLaunchKernelGGL(prefill_generic_kernel, dim3((unsigned)L, (unsigned)(B * Hq)), dim3(64), 0,
                     st, p);
  return check_launch("lq_int4_prefill_attention");
}
