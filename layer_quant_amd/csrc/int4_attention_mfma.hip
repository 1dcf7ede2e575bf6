// MFMA fast path of the INT4 decode attention (head_dim 128, group 32/64/128, bf16 queries).
//
// One workgroup = 4 waves on one (batch, KV head, key split); each wave walks its own key range
// in tiles of 32 keys and the 4 partial softmax states are merged through LDS at the end.
// Every packed KV byte and scale is read from HBM once per (batch, KV head): the NREP query
// heads that share a KV head are columns of the same MFMA tile.
//
// MFMA v_mfma_f32_16x16x32_bf16, D[16x16] += A[16x32] * B[32x16]. Lane l holds A row l%16 and
// B column l%16, each with K slots 8*(l/16) .. +7, and D rows 4*(l/16) .. +3 of column l%16.
//
// Columns. The 16 columns are (group m, head h) pairs, j = m*NREP + h, NREP*(128/g) <= 16.
//
// QK^T. Lane (q, r) loads the 16-byte unit q (dims 32q .. 32q+31) of key row r with one dwordx4
// and feeds dword c of it to MFMA c (A = 16 keys x 32 K slots). B = the matching query dims,
// placed only in the columns whose group m owns them (zero elsewhere), so after the 4 MFMAs
// column (m, h) holds the group-m partial dot product of head h; scaling by the key scale of
// group m and summing the columns of equal h (DPP row rotations) gives the score of head h.
// Nibbles decode in registers to bf16 with a magic number: bits 0x4300 | (n ^ 8) are the value
// 136 + n, so the accumulator starts at -136 * sum(q) of the column's dims.
//
// P V. A = V^T: 16 dims x 32 keys, B = P' with P'[key][(m, h)] = p[key][h] * vscale[key][m].
// Lane (q, c) needs dword c of key rows q + 4e (e = 0..7), so MFMA k (k = 0..7) covers dims
// 8c + k. The V rows arrive as 128-bit loads (32-bit loads cap the stream near 4.2 TB/s on MI355X
// against 7 TB/s for 128-bit) and pass through a per-wave LDS buffer into that layout; the output
// column (m, h) is kept only for dims of group m. P' is split into bf16 hi + lo (two MFMAs, about
// 16 significant bits). The value offset 136 of the V decode is removed at the end with
// sum_keys P' from one more MFMA against a ones operand.
#include <math.h>
#include <stdlib.h>

#include "int4_attention.h"

namespace lq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int FAST_D = 128;
constexpr int SUB = 32;              // keys per MFMA sub-tile (the K depth of the P V product)
constexpr int NSUB = 1;              // sub-tiles per iteration; one softmax max per iteration
constexpr int TILE = SUB * NSUB;     // keys per wave iteration
constexpr int WAVES = 4;
constexpr float LAZY_LOG2 = 8.0f;    // running-max slack of the lazy softmax rescale
constexpr uint32_t NIB2 = 0x000F000Fu;
constexpr int BUF_DWORD3 = 0x00020000;  // raw 32-bit buffer, gfx9 family
// Non-temporal (streaming) loads of the packed K/V rows and scales: each byte is read once per
// call, and at B=64, ctx 16384 the 1.34 GB stream measured 248 us with the default policy and
// 237 us with nt (a read-only probe of the same volume: 7.2 TB/s with nt, 5.4-6.3 without).
constexpr int KV_LOAD_POLICY = 2;

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x4_t mfma_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// One bf16 pair from two nibbles of x (bits 3:0 and 19:16, two's complement): the nibble xor 8
// in the mantissa of bf16 128.0, i.e. the value 136 + n. The expression compiles to a single
// v_bitop3_b32 on gfx950.
__device__ __forceinline__ uint32_t nib_pair(uint32_t x) {
  return ((x ^ 0x00080008u) & NIB2) | 0x43004300u;
}

// 8 nibbles of one dword -> bf16 values 136 + n, in the slot order of dims (0, 4, 1, 5, 2, 6, 3, 7).
__device__ __forceinline__ u32x4_t decode_k(uint32_t w) {
  u32x4_t o;
  o.x = nib_pair(w);
  o.y = nib_pair(w >> 4);
  o.z = nib_pair(w >> 8);
  o.w = nib_pair(w >> 12);
  return o;
}

// a * b summed over the columns that share a query head: columns j = m*NREP + h, unused columns
// hold 0. Row rotations by 8, 4, 2, 1 lanes; with contraction off each level is one
// v_add_f32_dpp (a fused multiply-add cannot take the DPP operand and would need a separate move).
template <int NREP>
__device__ __forceinline__ float column_sum(float a, float b) {
#pragma clang fp contract(off)
  float x = a * b;
  if constexpr (NREP <= 8) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, true));
  if constexpr (NREP <= 4) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, true));
  if constexpr (NREP <= 2) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, true));
  if constexpr (NREP <= 1) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, true));
  return x;
}

template <int G>
struct TileRegs {
  u32x4_t kq[NSUB][2];      // [sub][16-key half]: 16-byte unit l/16 (dims 32*(l/16) ..) of row l%16
  u32x4_t vq[NSUB][2];      // [sub][16-key half]: 16-byte unit l%4 of V row l/4
  float ksr[G];             // key / value scales of key row l%32, staged through LDS
  float vsr[G];
};

// G consecutive fp32 scale words at byte offset off, as one buffer load. (The words are
// reinterpreted with __uint_as_float: with this compiler, __builtin_bit_cast(float, w[m]) of a
// vector element narrowed the 128-bit load to its first dword and lost the other three.)
template <int G>
__device__ __forceinline__ void load_scales(__amdgpu_buffer_rsrc_t r, int off, float (&v)[G]) {
  if constexpr (G == 4) {
    const u32x4_t w = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, KV_LOAD_POLICY);
#pragma unroll
    for (int m = 0; m < 4; ++m) v[m] = __uint_as_float(w[m]);
  } else if constexpr (G == 2) {
    const u32x2_t w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, KV_LOAD_POLICY);
    v[0] = __uint_as_float(w[0]);
    v[1] = __uint_as_float(w[1]);
  } else {
    v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, KV_LOAD_POLICY));
  }
}

// Per-wave bases of this (batch, KV head) block; rows are contiguous (64 packed bytes, G scale
// words). Each tile builds buffer descriptors whose base is the tile's first key and whose size
// ends at key S, so the hardware range check (vector + immediate offset; the scalar offset is
// kept 0 because it is not range-checked) returns 0 for keys past S.
struct Rsrc {
  const uint8_t* kb;
  const uint8_t* vb;
  const float* ksb;
  const float* vsb;
  int kvo, vvo, svo;  // per-lane byte offsets inside a tile (K unit, V unit, scale row)
};

template <int G>
__device__ __forceinline__ void load_tile(const Rsrc& R, int tb, int S, TileRegs<G>& r) {
  tb = __builtin_amdgcn_readfirstlane(tb);  // uniform by construction; lets the descriptors live in SGPRs
  const int rem = S - tb;  // > 0
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)(R.kb + (int64_t)tb * 64), 0, rem * 64, BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)(R.vb + (int64_t)tb * 64), 0, rem * 64, BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t rks = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(R.ksb + (int64_t)tb * G), 0, rem * G * 4, BUF_DWORD3);
  const __amdgpu_buffer_rsrc_t rvs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(R.vsb + (int64_t)tb * G), 0, rem * G * 4, BUF_DWORD3);
  load_scales<G>(rks, R.svo, r.ksr);  // lanes l and l + 32 read the same row
  load_scales<G>(rvs, R.svo, r.vsr);
#pragma unroll
  for (int sb = 0; sb < NSUB; ++sb) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      r.kq[sb][t] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, R.kvo + (SUB * sb + 16 * t) * 64, 0, KV_LOAD_POLICY));
      r.vq[sb][t] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rv, R.vvo + (SUB * sb + 16 * t) * 64, 0, KV_LOAD_POLICY));
    }
  }
}

template <int NREP, int G>
__global__ __launch_bounds__(256) void attn_fast_kernel(AttnParams p) {
  constexpr int NCOL = NREP * G;
  constexpr int CPG = 4 / G;  // 32-dim chunks per group
  static_assert(NCOL <= 16, "columns exceed the MFMA tile");
  __shared__ float sc_lds[WAVES][2][2][G][TILE];  // [wave][buffer][k/v][group][key]
  __shared__ u32x4_t v_lds[WAVES][TILE][4];         // [wave][key][16-byte unit]: one V tile
  __shared__ float o_lds[WAVES][NREP][FAST_D];
  __shared__ float ml_lds[WAVES][2][NREP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q4 = lane >> 4;
  const int c16 = lane & 15;
  const int unit = blockIdx.x;
  const int split = blockIdx.y;
  const int b = unit / p.Hkv;
  const int kvh = unit - b * p.Hkv;
  const int S = (int)p.S;
  const int t0 = split * (int)p.chunk;
  const int t1 = min(S, t0 + (int)p.chunk);
  const int tpw = (int)p.chunk / WAVES;
  const int w0 = t0 + wave * tpw;
  const int w1 = min(t1, w0 + tpw);

  const bool colvalid = c16 < NCOL;
  const int colh = c16 % NREP;
  const int colm = colvalid ? c16 / NREP : 0;

  // Query operands. Lane (q, .) feeds MFMA c with dword c of its key unit q, i.e. dims
  // 32q + 8c .. 32q + 8c + 7 (slot order kPerm); the query is placed only in the columns whose
  // group owns those dims, so each column accumulates exactly its group's partial dot product.
  const uint16_t* qbits = (const uint16_t*)p.q.data;
  const int64_t qbase = b * p.q.s[0] + (int64_t)(kvh * NREP + colh) * p.q.s[1];
  constexpr int kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  const bool use = colvalid && (q4 / CPG == colm);
  u32x4_t qop[4];
  float qsum = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t lo = 0, hi = 0;
      if (use) {
        lo = qbits[qbase + (32 * q4 + 8 * c + kPerm[2 * u]) * p.q.s[2]];
        hi = qbits[qbase + (32 * q4 + 8 * c + kPerm[2 * u + 1]) * p.q.s[2]];
      }
      qsum += bf16_bits_to_float(lo) + bf16_bits_to_float(hi);
      qop[c][u] = lo | (hi << 16);
    }
  }
  qsum += __shfl_xor(qsum, 16, 64);
  qsum += __shfl_xor(qsum, 32, 64);
  const float cinit = -136.0f * qsum;

  Rsrc R;
  R.kb = p.kp + b * p.kps[0] + kvh * p.kps[1];
  R.vb = p.vp + b * p.vps[0] + kvh * p.vps[1];
  R.ksb = p.ks + b * p.kss[0] + kvh * p.kss[1];
  R.vsb = p.vs + b * p.vss[0] + kvh * p.vss[1];
  // QK A-row i of a 16-key half is key 4 (i & 3) + (i >> 2), so that output row 4q + r (held by
  // lane group q) is key 4r + q, and lane group q's 8 keys of a 32-key sub-tile are q + 4e
  // (e = 4t + r): the V loads of key slot e then cover keys 4e .. 4e+3 contiguously.
  R.kvo = (4 * (c16 & 3) + (c16 >> 2)) * 64 + 16 * q4;
  R.vvo = (lane >> 2) * 64 + 16 * (lane & 3);
  R.svo = (lane & 31) * G * 4;

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x4_t acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t corr = {0.0f, 0.0f, 0.0f, 0.0f};
  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  // Scales of a tile go to LDS, transposed to [group][key] with log2(e)/sqrt(D) folded into the
  // key scales, one tile before their use; buffer (tile index & 1).
  auto stage_scales = [&](const TileRegs<G>& r, const int buf) {
    if (lane < TILE) {
      const int tok = lane;
      // key 16t + 4r + q is read by lane group q as element r: store it at 16t + 4q + r
      const int pos = (tok & ~15) | ((tok & 3) << 2) | ((tok >> 2) & 3);
#pragma unroll
      for (int m = 0; m < G; ++m) {
        sc_lds[wave][buf][0][m][pos] = r.ksr[m] * p.scale_sm;
        sc_lds[wave][buf][1][m][pos] = r.vsr[m];
      }
    }
  };

  auto process = [&](const int tb, const TileRegs<G>& cur, const TileRegs<G>& next,
                     const bool has_next) {
    const int buf = ((tb - w0) / TILE) & 1;
    if (has_next) stage_scales(next, buf ^ 1);
    // scores: per sub-tile 2 halves of 16 keys, 4 chunks each
    f32x4_t sacc[NSUB][2];
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      sacc[sb][0] = f32x4_t{cinit, cinit, cinit, cinit};
      sacc[sb][1] = sacc[sb][0];
      // the two 16-key halves are independent chains: interleave them
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          sacc[sb][t] = mfma_bf16(decode_k(cur.kq[sb][t][c]), qop[c], sacc[sb][t]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();

    // key slot e of sub-tile sb (e = 4t + r) is key tb + 32 sb + 16 t + 4 r + (l/16)
    float s[NSUB][8];
    f32x4_t vsc[NSUB][2];
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f32x4_t ks4 = *(const f32x4_t*)&sc_lds[wave][buf][0][colm][SUB * sb + 16 * t + 4 * q4];
        vsc[sb][t] = *(const f32x4_t*)&sc_lds[wave][buf][1][colm][SUB * sb + 16 * t + 4 * q4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[sb][4 * t + r] = column_sum<NREP>(sacc[sb][t][r], ks4[r]);
      }
    }
    if (p.mask != nullptr) {
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int tok = tb + SUB * sb + 16 * (e >> 2) + 4 * (e & 3) + q4;
          s[sb][e] += (tok < p.mask_len) ? p.mask[b * p.mask_sb + (int64_t)tok * p.mask_sk]
                                         : -INFINITY;
        }
      }
    }
    if (tb + TILE > w1) {
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int tok = tb + SUB * sb + 16 * (e >> 2) + 4 * (e & 3) + q4;
          s[sb][e] = tok < w1 ? s[sb][e] : -INFINITY;
        }
      }
    }
    // Lazy rescaling: p = 2^(s - m_run) with a running max that only moves when a score exceeds
    // it by more than LAZY_LOG2 (p <= 2^LAZY_LOG2 otherwise), so the cross-lane max and the
    // accumulator rescale leave the common path. The first tile always takes the update.
    float lm = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
#pragma unroll
      for (int e = 0; e < 8; ++e) lm = fmaxf(lm, s[sb][e]);
    }
    if (__any(lm > m_run + LAZY_LOG2)) {
      float mt = fmaxf(lm, __shfl_xor(lm, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run, mt);
      // acc and l are still zero while m_run is -inf: no rescale needed then
      const float alpha = (m_run == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      if (alpha != 1.0f) {
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] *= alpha;
        corr *= alpha;
        l_run *= alpha;
      }
      m_run = m_new;
    }
    // m_run is -inf only while every score so far is -inf; a finite stand-in keeps
    // exp2(-inf - m) = 0 without a per-score select (a finite score takes the update above)
    const float m_use = fmaxf(m_run, -3.0e38f);
    float psum = 0.0f;
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s[sb][e] = __builtin_amdgcn_exp2f(s[sb][e] - m_use);
        psum += s[sb][e];
      }
    }
    l_run += psum;

#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      // P' = p * vscale, split into bf16 hi + lo
      u32x4_t bhi, blo;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = 2 * u;
        const float a0 = s[sb][e] * vsc[sb][e >> 2][e & 3];
        const float a1 = s[sb][e + 1] * vsc[sb][(e + 1) >> 2][(e + 1) & 3];
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a0, a1}, bf16x2_t));
        const float r0 = a0 - __builtin_bit_cast(float, h << 16);
        const float r1 = a1 - __builtin_bit_cast(float, h & 0xffff0000u);
        bhi[u] = h;
        blo[u] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t));
      }
      // V rows through this wave's LDS buffer: dword c16 of key rows q4 + 4e (e = 0..7)
#pragma unroll
      for (int t = 0; t < 2; ++t) v_lds[wave][16 * t + (lane >> 2)][lane & 3] = cur.vq[sb][t];
      const uint32_t* vrow = (const uint32_t*)&v_lds[wave][0][0];
      uint32_t vw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) vw[e] = vrow[(q4 + 4 * e) * 16 + c16];
      // V decode: pair the key slots (2u, 2u+1), nibble k of each dword -> MFMA k
      uint32_t ylo[4], yhi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        ylo[u] = __builtin_amdgcn_perm(vw[2 * u + 1], vw[2 * u], 0x05040100u);
        yhi[u] = __builtin_amdgcn_perm(vw[2 * u + 1], vw[2 * u], 0x07060302u);
      }
      // four dims-sets at a time: their hi products, then their lo products, so that the two
      // MFMAs into one accumulator are separated by three independent ones
#pragma unroll
      for (int k0 = 0; k0 < 8; k0 += 4) {
        u32x4_t a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int u = 0; u < 4; ++u) a[j][u] = nib_pair((k0 < 4 ? ylo[u] : yhi[u]) >> (4 * j));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[k0 + j] = mfma_bf16(a[j], bhi, acc[k0 + j]);
        if (k0 == 0) corr = mfma_bf16(ones, bhi, corr);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[k0 + j] = mfma_bf16(a[j], blo, acc[k0 + j]);
        if (k0 == 4) corr = mfma_bf16(ones, blo, corr);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // three register stages: two tiles of loads stay in flight while a third is processed (a
  // fourth stage measured the same)
  TileRegs<G> ra, rb, rc;
  if (w0 < w1) {
    load_tile<G>(R, w0, S, ra);
    stage_scales(ra, 0);
  }
  if (w0 + TILE < w1) load_tile<G>(R, w0 + TILE, S, rb);
  for (int tb = w0; tb < w1; tb += 3 * TILE) {
    if (tb + 2 * TILE < w1) load_tile<G>(R, tb + 2 * TILE, S, rc);
    process(tb, ra, rb, tb + TILE < w1);
    if (tb + TILE >= w1) break;
    if (tb + 3 * TILE < w1) load_tile<G>(R, tb + 3 * TILE, S, ra);
    process(tb + TILE, rb, rc, tb + 2 * TILE < w1);
    if (tb + 2 * TILE >= w1) break;
    if (tb + 4 * TILE < w1) load_tile<G>(R, tb + 4 * TILE, S, rb);
    process(tb + 2 * TILE, rc, ra, tb + 3 * TILE < w1);
  }

  // per-wave partial -> LDS
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  const bool own = colvalid && (q4 / CPG == colm);
  if (own) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o_lds[wave][colh][32 * q4 + 8 * r + k] = acc[k][r] - 136.0f * corr[r];
      }
    }
  }
  if (lane < NREP) {
    ml_lds[wave][0][lane] = m_run;
    ml_lds[wave][1][lane] = l_run;
  }
  __syncthreads();

  // merge the 4 waves
  for (int idx = tid; idx < NREP * FAST_D; idx += 256) {
    const int h = idx / FAST_D;
    const int d = idx - h * FAST_D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, ml_lds[w][0][h]);
    float L = 0.0f;
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float mw = ml_lds[w][0][h];
      const float wt = (mw == -INFINITY) ? 0.0f : exp2f(mw - M);
      L += wt * ml_lds[w][1][h];
      a += wt * o_lds[w][h][d];
    }
    const int qh = kvh * NREP + h;
    if (p.nsplit == 1) {
      store_float(p.out.data, p.out.dtype, b * p.out.s[0] + qh * p.out.s[1] + d * p.out.s[2],
                  a / L);
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + qh) * p.nsplit + split;
      p.ws_acc[slot * FAST_D + d] = a;
      if (d == 0) {
        p.ws_m[slot] = M;
        p.ws_l[slot] = L;
      }
    }
  }
}

bool fast_path_shape_ok(int64_t head_dim, int group_size, int64_t n_q_heads,
                        int64_t n_kv_heads) {
  if (head_dim != FAST_D) return false;
  if (group_size != 32 && group_size != 64 && group_size != 128) return false;
  if (n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0) return false;
  const int64_t nrep = n_q_heads / n_kv_heads;
  if (nrep != 1 && nrep != 2 && nrep != 4 && nrep != 8 && nrep != 16) return false;
  return nrep * (FAST_D / group_size) <= 16;
}

static bool force_generic() {
  static const int v = [] {
    const char* e = getenv("LQ_ATTN_FORCE_GENERIC");
    return (e != nullptr && e[0] == '1') ? 1 : 0;
  }();
  return v != 0;
}

bool fast_path_ok(const AttnParams& p) {
  if (force_generic()) return false;
  if (!fast_path_shape_ok(p.D, p.g, p.Hq, p.Hkv)) return false;
  if (p.q.dtype != LQ_BF16) return false;
  // contiguous key rows: 64 packed bytes per key, D/g scale words per key
  const int64_t G = FAST_D / p.g;
  if (p.kps[3] != 1 || p.vps[3] != 1 || p.kps[2] != 64 || p.vps[2] != 64) return false;
  if (p.kss[3] != 1 || p.vss[3] != 1 || p.kss[2] != G || p.vss[2] != G) return false;
  const int64_t strides[4] = {p.kps[0], p.kps[1], p.vps[0], p.vps[1]};
  for (int64_t s : strides) {
    if (s % 4 != 0) return false;
  }
  if (((uintptr_t)p.kp & 3) != 0 || ((uintptr_t)p.vp & 3) != 0) return false;
  if (((uintptr_t)p.ks & 3) != 0 || ((uintptr_t)p.vs & 3) != 0) return false;
  // buffer sizes of one (batch, KV head) block are 32-bit
  if (p.S * 64 >= ((int64_t)1 << 31)) return false;
  return true;
}

// Waves of attn_fast_kernel resident on the current device at once: its register use (over 128
// VGPRs) leaves 2 waves per SIMD, 4 SIMDs per CU.
static int64_t resident_fast_waves() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 2048;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    cached[dev] = cus * 4 * 2;
  }
  return cached[dev];
}

SplitPlan plan_fast(int64_t B, int64_t Hkv, int64_t S) {
  // One resident generation of waves: each wave walks as many keys as that takes (rounded to the
  // 32-key tile, 4 waves per workgroup split). Fewer, longer waves amortize the per-wave setup
  // and the 4-wave merge, and at B * Hkv >= resident / 4 no split-K merge runs at all.
  const int64_t target_waves = resident_fast_waves();
  int64_t tpw = (B * Hkv * S + target_waves - 1) / target_waves;
  tpw = ((tpw + TILE - 1) / TILE) * TILE;
  tpw = std::min<int64_t>(std::max<int64_t>(tpw, TILE), (int64_t)1 << 20);
  SplitPlan sp{};
  sp.chunk = WAVES * tpw;
  sp.nsplit = (int)std::max<int64_t>(1, (S + sp.chunk - 1) / sp.chunk);
  return sp;
}

template <int NREP, int G>
static void launch_one(const AttnParams& p, hipStream_t st) {
  hipLaunchKernelGGL((attn_fast_kernel<NREP, G>), dim3((unsigned)(p.B * p.Hkv), (unsigned)p.nsplit),
                     dim3(256), 0, st, p);
}

int launch_fast(const AttnParams& p, hipStream_t st) {
  const int G = FAST_D / p.g;
  switch (p.nrep * 100 + G) {
    case 104: launch_one<1, 4>(p, st); break;
    case 204: launch_one<2, 4>(p, st); break;
    case 404: launch_one<4, 4>(p, st); break;
    case 102: launch_one<1, 2>(p, st); break;
    case 202: launch_one<2, 2>(p, st); break;
    case 402: launch_one<4, 2>(p, st); break;
    case 802: launch_one<8, 2>(p, st); break;
    case 101: launch_one<1, 1>(p, st); break;
    case 201: launch_one<2, 1>(p, st); break;
    case 401: launch_one<4, 1>(p, st); break;
    case 801: launch_one<8, 1>(p, st); break;
    case 1601: launch_one<16, 1>(p, st); break;
    default:
      return fail(LQ_ERR_UNSUPPORTED, "fast attention: no instance for nrep=%d groups=%d",
                  p.nrep, G);
  }
  return check_launch("lq_int4_decode_attention (mfma)");
}

}  // namespace lq
