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
// QK^T. A = 16 keys x 32 dims of one 32-dim chunk, B = the query dims of that chunk, placed only
// in the columns whose group m owns the chunk (zero elsewhere). Accumulating the 4 chunks gives,
// in column (m, h), the group-m partial dot product of head h; scaling by the key scale of group
// m and summing the columns of equal h (DPP row rotations) gives the score in every column of h.
// Nibbles decode in registers to bf16 with a magic number: bits 0x4300 | (n ^ 8) are the value
// 136 + n, so the accumulator starts at -136 * sum(q) of the column's dims.
//
// P V. A = V^T: 16 dims x 32 keys, B = P' with P'[key][(m, h)] = p[key][h] * vscale[key][m].
// Lane (q, c) loads dword c of 8 key rows, so MFMA k (k = 0..7) covers dims 8c + k; the output
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

constexpr int FAST_D = 128;
constexpr int TILE = 32;
constexpr int WAVES = 4;
constexpr uint32_t NIB2 = 0x000F000Fu;
constexpr int BUF_DWORD3 = 0x00020000;  // raw 32-bit buffer, gfx9 family

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

// sum over the columns that share a query head: columns j = m*NREP + h, unused columns hold 0
template <int NREP>
__device__ __forceinline__ float column_sum(float x) {
  if constexpr (NREP <= 8) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  if constexpr (NREP <= 4) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  if constexpr (NREP <= 2) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
  if constexpr (NREP <= 1) x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
  return x;
}

struct TileRegs {
  uint32_t kw[2][4];  // [16-key half][32-dim chunk]: dword (4*chunk + l/16) of key row l%16
  uint32_t vw[8];     // dword l%16 of the 8 key rows of this lane's K slots
  float ksr[2];       // key / value scale words, staged through LDS
  float vsr[2];
};

struct Rsrc {
  __amdgpu_buffer_rsrc_t k, v, ks, vs;
  int kvo, vvo, ksvo[2], vsvo[2];  // per-lane byte offsets
  int krow, vrow, ksrow, vsrow;  // byte strides of one key row
};

template <int G>
__device__ __forceinline__ void load_tile(const Rsrc& R, int tb, TileRegs& r) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int so = (tb + 16 * t) * R.krow;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      r.kw[t][c] = __builtin_amdgcn_raw_buffer_load_b32(R.k, R.kvo + 16 * c, so, 0);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int so = (tb + 16 * (e >> 2) + (e & 3)) * R.vrow;
    r.vw[e] = __builtin_amdgcn_raw_buffer_load_b32(R.v, R.vvo, so, 0);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (i * 64 < G * TILE) {
      r.ksr[i] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(R.ks, R.ksvo[i], tb * R.ksrow, 0));
      r.vsr[i] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(R.vs, R.vsvo[i], tb * R.vsrow, 0));
    }
  }
}

template <int NREP, int G>
__global__ __launch_bounds__(256) void attn_fast_kernel(AttnParams p) {
  constexpr int NCOL = NREP * G;
  constexpr int CPG = 4 / G;  // 32-dim chunks per group
  static_assert(NCOL <= 16, "columns exceed the MFMA tile");
  __shared__ float sc_lds[WAVES][2][G][TILE];
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

  // query operands of the 4 chunks and the column sums for the decode offset
  const uint16_t* qbits = (const uint16_t*)p.q.data;
  const int64_t qbase = b * p.q.s[0] + (int64_t)(kvh * NREP + colh) * p.q.s[1];
  constexpr int kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  u32x4_t qop[4];
  float qsum = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool use = colvalid && (c / CPG == colm);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t lo = 0, hi = 0;
      if (use) {
        lo = qbits[qbase + (32 * c + 8 * q4 + kPerm[2 * u]) * p.q.s[2]];
        hi = qbits[qbase + (32 * c + 8 * q4 + kPerm[2 * u + 1]) * p.q.s[2]];
      }
      qsum += bf16_bits_to_float(lo) + bf16_bits_to_float(hi);
      qop[c][u] = lo | (hi << 16);
    }
  }
  qsum += __shfl_xor(qsum, 16, 64);
  qsum += __shfl_xor(qsum, 32, 64);
  const float cinit = -136.0f * qsum;

  // buffer resources over this (batch, KV head); loads past the last key return 0
  Rsrc R;
  {
    const uint8_t* kb = p.kp + b * p.kps[0] + kvh * p.kps[1];
    const uint8_t* vb = p.vp + b * p.vps[0] + kvh * p.vps[1];
    const float* ksb = p.ks + b * p.kss[0] + kvh * p.kss[1];
    const float* vsb = p.vs + b * p.vss[0] + kvh * p.vss[1];
    R.krow = (int)p.kps[2];
    R.vrow = (int)p.vps[2];
    R.ksrow = (int)p.kss[2] * 4;
    R.vsrow = (int)p.vss[2] * 4;
    R.k = __builtin_amdgcn_make_buffer_rsrc((void*)kb, 0, (S - 1) * R.krow + 64, BUF_DWORD3);
    R.v = __builtin_amdgcn_make_buffer_rsrc((void*)vb, 0, (S - 1) * R.vrow + 64, BUF_DWORD3);
    R.ks = __builtin_amdgcn_make_buffer_rsrc(
        (void*)ksb, 0, ((S - 1) * (int)p.kss[2] + (G - 1) * (int)p.kss[3] + 1) * 4, BUF_DWORD3);
    R.vs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)vsb, 0, ((S - 1) * (int)p.vss[2] + (G - 1) * (int)p.vss[3] + 1) * 4, BUF_DWORD3);
    R.kvo = c16 * R.krow + 4 * q4;
    R.vvo = 4 * q4 * R.vrow + 4 * c16;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = lane + 64 * i;
      const int tok = idx / G;
      const int m = idx - tok * G;
      R.ksvo[i] = (tok * (int)p.kss[2] + m * (int)p.kss[3]) * 4;
      R.vsvo[i] = (tok * (int)p.vss[2] + m * (int)p.vss[3]) * 4;
    }
  }

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x4_t acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t corr = {0.0f, 0.0f, 0.0f, 0.0f};
  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  auto process = [&](const int tb, const TileRegs& cur) {
    // stage this tile's scales transposed, sc_lds[.][m][key]; fold log2(e)/sqrt(D) into K's
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = lane + 64 * i;
      if (idx < G * TILE) {
        const int tok = idx / G;
        const int m = idx - tok * G;
        sc_lds[wave][0][m][tok] = cur.ksr[i] * p.scale_sm;
        sc_lds[wave][1][m][tok] = cur.vsr[i];
      }
    }

    // scores: 2 halves of 16 keys, 4 chunks each
    f32x4_t sacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      sacc[t] = f32x4_t{cinit, cinit, cinit, cinit};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        sacc[t] = mfma_bf16(decode_k(cur.kw[t][c]), qop[c], sacc[t]);
      }
    }
    __builtin_amdgcn_wave_barrier();
    const f32x4_t ks0 = *(const f32x4_t*)&sc_lds[wave][0][colm][4 * q4];
    const f32x4_t ks1 = *(const f32x4_t*)&sc_lds[wave][0][colm][16 + 4 * q4];
    const f32x4_t vs0 = *(const f32x4_t*)&sc_lds[wave][1][colm][4 * q4];
    const f32x4_t vs1 = *(const f32x4_t*)&sc_lds[wave][1][colm][16 + 4 * q4];

    float s[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = column_sum<NREP>(sacc[0][r] * ks0[r]);
      s[4 + r] = column_sum<NREP>(sacc[1][r] * ks1[r]);
    }
    if (p.mask != nullptr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = tb + 16 * (e >> 2) + 4 * q4 + (e & 3);
        s[e] += (tok < p.mask_len) ? p.mask[b * p.mask_sb + (int64_t)tok * p.mask_sk] : -INFINITY;
      }
    }
    if (tb + TILE > w1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = tb + 16 * (e >> 2) + 4 * q4 + (e & 3);
        s[e] = tok < w1 ? s[e] : -INFINITY;
      }
    }
    float mt = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])),
                     fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    // acc and l are still zero while m_run is -inf: no rescale needed then
    const float alpha = (m_run == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float pe[8];
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pe[e] = (s[e] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s[e] - m_new);
      psum += pe[e];
    }
    l_run = l_run * alpha + psum;
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] *= alpha;
      corr *= alpha;
    }
    m_run = m_new;

    // P' = p * vscale, split into bf16 hi + lo
    u32x4_t bhi, blo;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = 2 * u;
      const float a0 = pe[e] * (e < 4 ? vs0[e] : vs1[e - 4]);
      const float a1 = pe[e + 1] * (e + 1 < 4 ? vs0[e + 1] : vs1[e - 3]);
      const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a0, a1}, bf16x2_t));
      const float r0 = a0 - __builtin_bit_cast(float, h << 16);
      const float r1 = a1 - __builtin_bit_cast(float, h & 0xffff0000u);
      bhi[u] = h;
      blo[u] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t));
    }

    // V decode: pair the key slots (2u, 2u+1), nibble k of each dword -> MFMA k
    uint32_t ylo[4], yhi[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ylo[u] = __builtin_amdgcn_perm(cur.vw[2 * u + 1], cur.vw[2 * u], 0x05040100u);
      yhi[u] = __builtin_amdgcn_perm(cur.vw[2 * u + 1], cur.vw[2 * u], 0x07060302u);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      u32x4_t a;
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = nib_pair((k < 4 ? ylo[u] : yhi[u]) >> (4 * (k & 3)));
      acc[k] = mfma_bf16(a, bhi, acc[k]);
      acc[k] = mfma_bf16(a, blo, acc[k]);
    }
    corr = mfma_bf16(ones, bhi, corr);
    corr = mfma_bf16(ones, blo, corr);
    __builtin_amdgcn_wave_barrier();
  };

  // two register stages, ping-pong: the next tile's loads are in flight during this tile's math
  TileRegs ra, rb;
  if (w0 < w1) load_tile<G>(R, w0, ra);
  for (int tb = w0; tb < w1; tb += 2 * TILE) {
    if (tb + TILE < w1) load_tile<G>(R, tb + TILE, rb);
    process(tb, ra);
    if (tb + TILE >= w1) break;
    if (tb + 2 * TILE < w1) load_tile<G>(R, tb + 2 * TILE, ra);
    process(tb + TILE, rb);
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
  if (p.kps[3] != 1 || p.vps[3] != 1) return false;
  const int64_t strides[6] = {p.kps[0], p.kps[1], p.kps[2], p.vps[0], p.vps[1], p.vps[2]};
  for (int64_t s : strides) {
    if (s % 4 != 0) return false;
  }
  if (((uintptr_t)p.kp & 3) != 0 || ((uintptr_t)p.vp & 3) != 0) return false;
  // byte offsets inside one (batch, KV head) block are 32-bit buffer offsets
  const int64_t lim = (int64_t)1 << 31;
  if (p.S * std::max(p.kps[2], p.vps[2]) >= lim) return false;
  if ((p.S * std::max(p.kss[2], p.vss[2]) + 4 * std::max(p.kss[3], p.vss[3])) * 4 >= lim) {
    return false;
  }
  if (p.kss[2] < 0 || p.kss[3] < 0 || p.vss[2] < 0 || p.vss[3] < 0 || p.kps[2] <= 0 ||
      p.vps[2] <= 0) {
    return false;
  }
  return true;
}

SplitPlan plan_fast(int64_t B, int64_t Hkv, int64_t S) {
  // about 16K waves: keys per wave rounded to the 32-key tile, 4 waves per workgroup split
  const int64_t target_waves = 16384;
  int64_t tpw = (B * Hkv * S + target_waves - 1) / target_waves;
  tpw = ((tpw + TILE - 1) / TILE) * TILE;
  tpw = std::min<int64_t>(std::max<int64_t>(tpw, TILE), 1024);
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
