// MFMA fast path of the INT4 decode attention (head_dim 128, group 32/64/128, bf16 queries).
//
// One workgroup = 4 waves on one (batch, KV head, key split); the split's 32-key tiles are dealt
// to the waves in turn (wave w takes tiles w, w + 4, ...) and the 4 partial softmax states are
// merged through LDS at the end.
// Every packed KV byte and scale is read from HBM once per (batch, KV head): the NREP query
// heads that share a KV head are columns of the same MFMA tile.
//
// Streaming. Each wave keeps a ring of 3 tile buffers in LDS filled by buffer loads that write
// LDS directly (16 bytes per lane, non-temporal): while tile i is computed, the loads of tiles
// i+1 and i+2 are in flight, with no registers held for them. This replaced a ring of register
// tiles (3 x 24 VGPRs per lane, V passed through LDS for its transpose anyway).
//
// Decode-token pack (lq_int4_decode_attention_pack). The wave whose last tile holds key S - 1
// quantises the new token's K and V rows with the pack kernel's code, writes them to cache row
// S - 1 and over that key's row in its LDS tile: one launch per layer instead of a pack launch
// and the attention.
//
// MFMA v_mfma_f32_16x16x32_bf16, D[16x16] += A[16x32] * B[32x16]. Lane l holds A row l%16 and
// B column l%16, each with K slots 8*(l/16) .. +7, and D rows 4*(l/16) .. +3 of column l%16.
//
// Columns. The 16 columns are (group m, head h) pairs, j = m*NREP + h, NREP*(128/g) <= 16.
//
// QK^T. Lane (q, r) reads the 16-byte unit q (dims 32q .. 32q+31) of key row r from LDS and
// feeds dword c of it to MFMA c (A = 16 keys x 32 K slots). B = the matching query dims,
// placed only in the columns whose group m owns them (zero elsewhere), so after the 4 MFMAs
// column (m, h) holds the group-m partial dot product of head h; scaling by the key scale of
// group m and summing the columns of equal h (DPP row rotations) gives the score of head h.
// Nibbles decode in registers to bf16 with a magic number: bits 0x4300 | (n ^ 8) are the value
// 136 + n, so the accumulator starts at -136 * sum(q) of the column's dims. Scores stay in raw
// units; log2(e)/sqrt(D) is applied inside the exponent's fused multiply-add.
//
// P V. A = V^T: 16 dims x 32 keys, B = P' with P'[key][(m, h)] = p[key][h] * vscale[key][m].
// Lane (q, c) reads dword c of key rows q + 4e (e = 0..7) from LDS, so MFMA k (k = 0..7) covers
// dims 8c + k; the output column (m, h) is kept only for dims of group m. P' is split into bf16
// hi + lo (two MFMAs, about 16 significant bits). Value nibbles decode into the top four mantissa
// bits of bf16 16.0, i.e. the value 24 + n, and the offset 24 is removed at the end with
// sum_keys P' from one more MFMA against a ones operand. The accumulators round at the magnitude
// of 24 * sum P' rather than of the result; decoded as 136 + n (the key decode above) the values
// gave an error about 5x larger, which dominated the kernel's error on outlier-channel data (a
// CPU emulation of both decodes, checked against the kernel on the same inputs, gave the ratio).
#include <math.h>
#include <stdlib.h>

#include "int4_attention.h"
#include "int4_quant.h"

namespace lq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int FAST_D = 128;
constexpr int TILE = 32;             // keys per wave iteration (the K depth of the P V product)
constexpr int WAVES = 4;             // waves per workgroup, each on its own key range
constexpr int THREADS = 64 * WAVES;
constexpr float LAZY_LOG2 = 8.0f;    // running-max slack of the lazy softmax rescale
constexpr uint32_t NIB2 = 0x000F000Fu;
constexpr int BUF_DWORD3 = 0x00020000;  // raw 32-bit buffer, gfx9 family
// The tile loads carry the non-temporal (nt) policy: each byte is read once per call, and at
// B=64, ctx 16384 the 1.34 GB stream measured 248 us with the default policy and 237 us with nt
// (a read-only probe of the same volume: 7.2 TB/s with nt, 5.4-6.3 without).

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

// One bf16 pair from two nibbles of x placed at bits 6:3 and 22:19: the nibble xor 8 in the top
// four mantissa bits of bf16 16.0, i.e. the value 24 + n (one v_bitop3_b32 after the shift that
// places the nibbles).
__device__ __forceinline__ uint32_t nib_pair_top(uint32_t x) {
  return ((x ^ 0x00400040u) & 0x00780078u) | 0x41804180u;
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

// One wave's copy of a 32-key tile in LDS, written by buffer loads that deliver straight to LDS
// (16 bytes per lane: lane l of one load writes bytes 16 l .. 16 l + 15 of its 1 KiB destination).
// K rows: 16-byte unit q of row r (r = key & 15 of the half) sits in slot 4 r + (q ^ ((r >> 2) & 3)),
// so that the 16 lanes of one row group of the QK reads hit 16 different slots modulo 16.
// V rows and the scales keep their HBM order ([key][64 bytes], [key][group]).
struct alignas(16) TileLds {
  u32x4_t k[2][64];
  u32x4_t v[2][64];
  float ks[TILE * 4];  // [key][group] (G <= 4)
  float vs[TILE * 4];
  float mk[TILE];      // additive mask of the tile's keys (masked calls only)
};

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor (base, stride 0, num_records = bytes, gfx9 dword 3) for wave-uniform
// arguments, so that it lives in 4 SGPRs.
__device__ __forceinline__ i32x4_t make_desc(const void* base, int bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4_t d;
  d[0] = (int32_t)(uint32_t)a;
  d[1] = (int32_t)((uint32_t)(a >> 32) & 0xffffu);
  d[2] = bytes;
  d[3] = BUF_DWORD3;
  return d;
}

// One 16-byte-per-lane buffer load that writes LDS directly: lane l's 16 bytes (at byte offset
// voff of the buffer; zero past num_records) land at LDS byte address lds + 16 l. Written as
// inline assembly with its own M0 set-up: the compiler's wait insertion for the builtin form did
// not track which LDS buffer each such load targets (it emitted no wait before the reads of one
// buffer and a full wait before the other's), so the waits are explicit (wait_loads) instead.
// M0 is declared clobbered; no other code of this kernel uses M0 (the compiler warns that a
// reserved register in a clobber list is not saved for it).
__device__ __forceinline__ void load_to_lds(i32x4_t desc, const void* lds, int voff) {
  const uint32_t addr =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds);
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen nt lds"
      :
      : "s"(addr), "v"(voff), "s"(desc)
      : "memory", "m0");
}

// The same with 4 bytes per lane (lane l's dword lands at lds + 4 l; each dword is range-checked
// on its own).
__device__ __forceinline__ void load_to_lds_b32(i32x4_t desc, const void* lds, int voff) {
  const uint32_t addr =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds);
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen nt lds"
      :
      : "s"(addr), "v"(voff), "s"(desc)
      : "memory", "m0");
}

// Wait until at most N vector-memory loads of this wave are outstanding (loads complete in issue
// order, so every load older than the newest N has landed).
template <int N>
__device__ __forceinline__ void wait_loads() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
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
  int kvo;  // this lane's source offset for the swizzled K slot
  const float* mb;     // mask row of this batch (masked calls)
  int msk_bytes;       // its key stride in bytes
  int64_t mask_len;    // keys the mask covers
};

// Loads issued per tile (and counted by the waits): K 2, V 2, scales 2, and the mask row.
template <bool MASK>
constexpr int tile_loads() { return MASK ? 7 : 6; }

// Issue the loads of the tile at key tb into B (2 for K, 2 for V, one each for the K and V
// scales on lanes below 8 G, and with MASK one for the tile's 32 mask values).
template <int G, bool MASK>
__device__ __forceinline__ void issue_tile(const Rsrc& R, int tb, int S, TileLds& B, int lane) {
  tb = __builtin_amdgcn_readfirstlane(tb);  // uniform by construction; descriptors in SGPRs
  const int rem = S - tb;  // > 0
  const i32x4_t rk = make_desc(R.kb + (int64_t)tb * 64, rem * 64);
  const i32x4_t rv = make_desc(R.vb + (int64_t)tb * 64, rem * 64);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    load_to_lds(rk, &B.k[h][0], R.kvo + 1024 * h);
    load_to_lds(rv, &B.v[h][0], 16 * lane + 1024 * h);
  }
  const i32x4_t rks = make_desc(R.ksb + (int64_t)tb * G, rem * G * 4);
  const i32x4_t rvs = make_desc(R.vsb + (int64_t)tb * G, rem * G * 4);
  // the tile's 32 G scale words of each kind: 16 bytes per lane on lanes 0..31 for G = 4, one
  // dword per lane on lanes below 32 G otherwise (16-byte units would straddle the end of the
  // scales at a ragged S); the other lanes are inactive and write nothing. issue_tile runs with
  // all 64 lanes active, so lane 0 always issues these two loads and every tile counts 6 loads
  // in the waits.
  if constexpr (G == 4) {
    if (lane < 32) {
      load_to_lds(rks, &B.ks[0], 16 * lane);
      load_to_lds(rvs, &B.vs[0], 16 * lane);
    }
  } else {
    if (lane < 32 * G) {
      load_to_lds_b32(rks, &B.ks[0], 4 * lane);
      load_to_lds_b32(rvs, &B.vs[0], 4 * lane);
    }
  }
  if constexpr (MASK) {
    // keys at or past the mask's length read 0 here and are set to -inf by the score code
    const int64_t mrem = R.mask_len - tb;
    const i32x4_t rm = make_desc(R.mb + (int64_t)tb * (R.msk_bytes >> 2),
                                 mrem > 0 ? (int)mrem * R.msk_bytes : 0);
    if (lane < TILE) load_to_lds_b32(rm, &B.mk[0], lane * R.msk_bytes);
  }
}

// Device-coherent (agent-scope, relaxed) store and load of a split-K partial: written through to
// where every XCD's L2 sees it, read past a possibly stale copy in this XCD's L2.
__device__ __forceinline__ void coherent_store(float* a, float v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The folded merge handles units with NREP * nsplit <= FOLD_MAX_PARTIALS: one thread's outputs
// then need at most 64 partial loads (128 at NREP = 1), all issued at once.
constexpr int FOLD_MAX_PARTIALS = 128;

// The merge of one (batch, KV head) unit's nsplit partials, by the unit's workgroup that arrived
// last, with the formulas of attn_merge_kernel: M = max_s m_s, w_s = 2^(m_s - M),
// out = sum_s w_s acc_s / sum_s w_s l_s. Every load goes out at once (thread t's acc partials of
// outputs t + 256 j over all splits; one (m, l) pair per thread for the first NREP * nsplit
// threads), so the merge costs one round trip of device-coherent loads. The weights are made once
// per (head, split) by those threads and shared through LDS, and every LDS walk over the splits is
// unrolled: computed per output, with a loop per split, the merge took 4-9 us of the kernel.
template <int NREP>
__device__ __forceinline__ void merge_unit(const AttnParams& p, int b, int kvh, float* s_w,
                                           float* s_wl, float* s_L) {
  constexpr int OPT = (NREP * FAST_D + THREADS - 1) / THREADS;  // outputs per thread
  constexpr int SMAX = FOLD_MAX_PARTIALS / NREP;                // splits at most
  const int tid = threadIdx.x;
  const int ns = p.nsplit;
  const int64_t head0 = (int64_t)b * p.Hq + kvh * NREP;
  float part[OPT][SMAX];
#pragma unroll
  for (int j = 0; j < OPT; ++j) {
    const int o = tid + THREADS * j;
    const int h = min(o / FAST_D, NREP - 1);
    const int d = o % FAST_D;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      part[j][s] = (s < ns) ? coherent_load(&p.ws_acc[((head0 + h) * ns + s) * FAST_D + d]) : 0.0f;
    }
  }
  // thread t < NREP * ns holds split s = t % ns of head h = t / ns ([h][s], h-major as in the
  // workspace); entries s >= ns of a head read a neighbour's slot (below FOLD_MAX_PARTIALS) and
  // are masked
  const bool owner = tid < NREP * ns;
  const int oh = owner ? tid / ns : 0;
  float mt = -INFINITY, lt = 0.0f;
  if (owner) {
    mt = coherent_load(&p.ws_m[head0 * ns + tid]);
    lt = coherent_load(&p.ws_l[head0 * ns + tid]);
    s_w[tid] = mt;
  }
  __syncthreads();
  float w = 0.0f;
  if (owner) {
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      const float ms = s_w[min(oh * ns + s, FOLD_MAX_PARTIALS - 1)];
      M = fmaxf(M, s < ns ? ms : -INFINITY);
    }
    w = (mt == -INFINITY) ? 0.0f : exp2f(mt - M);
    s_wl[tid] = w * lt;
  }
  __syncthreads();
  if (owner) {
    s_w[tid] = w;  // every read of the m values ended at the barrier above
    if (tid == oh * ns) {
      float L = 0.0f;
#pragma unroll
      for (int s = 0; s < SMAX; ++s) {
        const float wl = s_wl[min(oh * ns + s, FOLD_MAX_PARTIALS - 1)];
        L += s < ns ? wl : 0.0f;
      }
      s_L[oh] = L;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < OPT; ++j) {
    const int o = tid + THREADS * j;
    if (o >= NREP * FAST_D) break;
    const int h = o / FAST_D;
    const int d = o % FAST_D;
    float a = 0.0f;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      const float ws = s_w[min(h * ns + s, FOLD_MAX_PARTIALS - 1)];
      a += (s < ns ? ws : 0.0f) * part[j][s];
    }
    const int qh = kvh * NREP + h;
    store_float(p.out.data, p.out.dtype, b * p.out.s[0] + qh * p.out.s[1] + d * p.out.s[2],
                a / s_L[h]);
  }
}

template <int NREP, int G, bool MASK>
__global__ __launch_bounds__(THREADS) void attn_fast_kernel(AttnParams p) {
  constexpr int LPT = tile_loads<MASK>();
  constexpr int NCOL = NREP * G;
  constexpr int CPG = 4 / G;  // 32-dim chunks per group
  static_assert(NCOL <= 16, "columns exceed the MFMA tile");
  // 3 tile buffers per wave (separate LDS objects, one per ring position); a wave's partial
  // output and softmax state reuse its first buffer when they fit (NREP <= 8)
  constexpr bool O_IN_TILE = (NREP * FAST_D + 2 * NREP) * 4 <= (int)sizeof(TileLds);
  __shared__ TileLds tiles0[WAVES];
  __shared__ TileLds tiles1[WAVES];
  __shared__ TileLds tiles2[WAVES];
  __shared__ float o_sep[O_IN_TILE ? 1 : WAVES * (NREP * FAST_D + 2 * NREP)];

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
  // The workgroup's tiles are dealt to its waves in turn (wave w takes tiles w, w + 4, ...): the
  // four waves then read adjacent tiles, one stream per tensor per workgroup. With a contiguous
  // range per wave (four streams per tensor per workgroup) a read-only probe of this pattern ran
  // at 6.55 TB/s against 6.99 TB/s interleaved.
  const int ntile = (t1 - t0 + TILE - 1) / TILE;
  const int nw = ntile > wave ? (ntile - wave + WAVES - 1) / WAVES : 0;  // tiles of this wave
  auto tile_key = [&](const int i) { return t0 + (wave + WAVES * i) * TILE; };

  const bool colvalid = c16 < NCOL;
  const int colh = c16 % NREP;
  const int colm = colvalid ? c16 / NREP : 0;

  Rsrc R;
  R.kb = p.kp + b * p.kps[0] + kvh * p.kps[1];
  R.vb = p.vp + b * p.vps[0] + kvh * p.vps[1];
  R.ksb = p.ks + b * p.kss[0] + kvh * p.kss[1];
  R.vsb = p.vs + b * p.vss[0] + kvh * p.vss[1];
  // K slot l of a half holds row l >> 2, unit (l & 3) ^ ((l >> 4) & 3)
  R.kvo = (lane >> 2) * 64 + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
  R.mb = MASK ? p.mask + b * p.mask_sb : nullptr;
  R.msk_bytes = (int)(p.mask_sk * 4);
  R.mask_len = p.mask_len;

  // the first tiles' loads go out before the query set-up
  if (nw > 0) issue_tile<G, MASK>(R, tile_key(0), S, tiles0[wave], lane);
  if (nw > 1) issue_tile<G, MASK>(R, tile_key(1), S, tiles1[wave], lane);

  // Query operands. Lane (q, .) feeds MFMA c with dword c of its key unit q, i.e. dims
  // 32q + 8c .. 32q + 8c + 7 (slot order kPerm); the query is placed only in the columns whose
  // group owns those dims, so each column accumulates exactly its group's partial dot product.
  const uint16_t* qbits = (const uint16_t*)p.q.data;
  const int64_t qbase = b * p.q.s[0] + (int64_t)(kvh * NREP + colh) * p.q.s[1];
  constexpr int kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  const bool use = colvalid && (q4 / CPG == colm);
  // Every lane loads its 32 values (the address is valid for every lane) and the unused ones are
  // zeroed afterwards: loaded under `use`, each pair became a branch with its own wait.
  uint32_t qraw[4][8];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int k = 0; k < 8; ++k) qraw[c][k] = qbits[qbase + (32 * q4 + 8 * c + kPerm[k]) * p.q.s[2]];
  }
  u32x4_t qop[4];
  float qsum = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t lo = use ? qraw[c][2 * u] : 0u;
      const uint32_t hi = use ? qraw[c][2 * u + 1] : 0u;
      qsum += bf16_bits_to_float(lo) + bf16_bits_to_float(hi);
      qop[c][u] = lo | (hi << 16);
    }
  }
  qsum += __shfl_xor(qsum, 16, 64);
  qsum += __shfl_xor(qsum, 32, 64);
  const float cinit = -136.0f * qsum;
  const float csm = p.scale_sm;  // raw scores -> log2 units
  const float inv_csm = 1.0f / csm;

  // Fused pack (lq_int4_decode_attention_pack): the wave whose dealt tiles hold key S - 1 (its
  // last tile) loads the new token's K and V values here (lane j: dims 2j and 2j + 1) and packs
  // them when it reaches that tile, after the tile's wait (a full one, the last tile having no
  // loads behind it): the pack kernel's arithmetic, written to cache row S - 1 and over the key's
  // row in the LDS tile, whichever version the tile's loads read. (The fast path's caches have
  // 64-byte rows and contiguous scales, so the row is indexed directly.)
  constexpr int GH = FAST_D / (2 * G);  // lanes per quantisation group
  int pack_i = -1;                      // the wave's tile index holding key S - 1, or -1
  float kx0 = 0.0f, kx1 = 0.0f, vx0 = 0.0f, vx1 = 0.0f;
  if (p.pack && t1 == S) {
    const int tile = (S - 1 - t0) / TILE;
    if (tile % WAVES == wave) {
      pack_i = tile / WAVES;
      const int64_t kx = b * p.knew.s[0] + (int64_t)kvh * p.knew.s[1];
      const int64_t vx = b * p.vnew.s[0] + (int64_t)kvh * p.vnew.s[1];
      uint32_t sh[4];
      const uint32_t w0 = elem_word(p.knew.data, p.knew.dtype, kx + 2 * lane * p.knew.s[2], sh[0]);
      const uint32_t w1 = elem_word(p.knew.data, p.knew.dtype, kx + (2 * lane + 1) * p.knew.s[2], sh[1]);
      const uint32_t w2 = elem_word(p.vnew.data, p.vnew.dtype, vx + 2 * lane * p.vnew.s[2], sh[2]);
      const uint32_t w3 = elem_word(p.vnew.data, p.vnew.dtype, vx + (2 * lane + 1) * p.vnew.s[2], sh[3]);
      kx0 = word_elem(w0, sh[0], p.knew.dtype);
      kx1 = word_elem(w1, sh[1], p.knew.dtype);
      vx0 = word_elem(w2, sh[2], p.vnew.dtype);
      vx1 = word_elem(w3, sh[3], p.vnew.dtype);
    }
  }

  // QK A-row i of a 16-key half is key 4 (i & 3) + (i >> 2), so that output row 4q + r (held by
  // lane group q) is key 4r + q, and lane group q's 8 keys of the tile are q + 4e (e = 4t + r).
  const int krow = 4 * (c16 & 3) + (c16 >> 2);
  const int kslot = 4 * krow + (q4 ^ (c16 & 3));

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x4_t acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  f32x4_t corr = {0.0f, 0.0f, 0.0f, 0.0f};
  const u32x4_t ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};

  // Before the reads of the wave's tile i: wait for its loads, leaving the already issued loads
  // of its following tiles (LPT each) in flight.
  auto wait_tile = [&](const int i) {
    if (i + 2 < nw) wait_loads<2 * LPT>();
    else if (i + 1 < nw) wait_loads<LPT>();
    else wait_loads<0>();
  };

  auto process = [&](const int i, TileLds& B) {
    const int tb = tile_key(i);
    wait_tile(i);
    if (i == pack_i) {  // key S - 1 of this tile: the fused pack (LDS layout as in TileLds)
      float kscl, vscl;
      const uint32_t kbyte = int4_quantize_pair<GH>(kx0, kx1, kscl);
      const uint32_t vbyte = int4_quantize_pair<GH>(vx0, vx1, vscl);
      const int key = S - 1 - tb;
      const int hk = key >> 4;
      const int r = key & 15;
      ((uint8_t*)&B.k[hk][4 * r + ((lane >> 4) ^ ((r >> 2) & 3))])[lane & 15] = (uint8_t)kbyte;
      ((uint8_t*)&B.v[hk][0])[r * 64 + lane] = (uint8_t)vbyte;
      const_cast<uint8_t*>(R.kb)[(int64_t)(S - 1) * 64 + lane] = (uint8_t)kbyte;
      const_cast<uint8_t*>(R.vb)[(int64_t)(S - 1) * 64 + lane] = (uint8_t)vbyte;
      if ((lane & (GH - 1)) == 0) {
        B.ks[key * G + lane / GH] = kscl;
        B.vs[key * G + lane / GH] = vscl;
        const_cast<float*>(R.ksb)[(int64_t)(S - 1) * G + lane / GH] = kscl;
        const_cast<float*>(R.vsb)[(int64_t)(S - 1) * G + lane / GH] = vscl;
      }
    }
    // scores S^T (keys x columns) in raw units: two 16-key halves, 4 chunks each
    f32x4_t sacc[2];
    sacc[0] = f32x4_t{cinit, cinit, cinit, cinit};
    sacc[1] = sacc[0];
    u32x4_t kq[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) kq[t] = B.k[t][kslot];
    // Wave priority 1 over the MFMA sections (QK with the V decode, and P' with P V): of the two
    // waves on a SIMD, the one issuing MFMAs goes first and the other's softmax VALU work fills
    // the MFMA pipe's busy cycles. In one cold sweep at B=64, ctx 16384: 242-245 us without,
    // 230-233 us with; P V alone 243-248, QK alone 238-240.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int t = 0; t < 2; ++t) sacc[t] = mfma_bf16(decode_k(kq[t][c]), qop[c], sacc[t]);
    }
    // V operands, decoded here (they do not depend on the scores) so that this VALU work shares
    // a basic block with the QK MFMAs above: dword c16 of key rows q4 + 4e (e = 0..7), key slots
    // (2u, 2u+1) paired, nibble k of each dword -> MFMA k
    u32x4_t va[8];
    {
      const uint32_t* vrow = (const uint32_t*)&B.v[0][0];
      uint32_t vw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) vw[e] = vrow[(q4 + 4 * e) * 16 + c16];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t ylo = __builtin_amdgcn_perm(vw[2 * u + 1], vw[2 * u], 0x05040100u);
        const uint32_t yhi = __builtin_amdgcn_perm(vw[2 * u + 1], vw[2 * u], 0x07060302u);
        va[0][u] = nib_pair_top(ylo << 3);
        va[4][u] = nib_pair_top(yhi << 3);
#pragma unroll
        for (int j = 1; j < 4; ++j) {
          va[j][u] = nib_pair_top(ylo >> (4 * j - 3));
          va[4 + j][u] = nib_pair_top(yhi >> (4 * j - 3));
        }
      }
      // keep the decode here: without this the compiler sinks it past the softmax branches to
      // its use in the P V products
#pragma unroll
      for (int k = 0; k < 8; ++k) asm volatile("" : "+v"(va[k]));
    }

    __builtin_amdgcn_s_setprio(0);
    // key slot e (e = 4t + r) is key tb + 16 t + 4 r + (l/16)
    float s[8], vsc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = 16 * (e >> 2) + 4 * (e & 3) + q4;
      s[e] = column_sum<NREP>(sacc[e >> 2][e & 3], B.ks[key * G + colm]);
      vsc[e] = B.vs[key * G + colm];
    }
    if constexpr (MASK) {  // additive mask in raw score units; keys past its length are -inf
      float mv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) mv[e] = B.mk[16 * (e >> 2) + 4 * (e & 3) + q4];
      if (tb + TILE <= p.mask_len) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = fmaf(mv[e], inv_csm, s[e]);
      } else {
        const int mlim = (int)max<int64_t>(p.mask_len - tb, 0);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = 16 * (e >> 2) + 4 * (e & 3) + q4;
          s[e] = key < mlim ? fmaf(mv[e], inv_csm, s[e]) : -INFINITY;
        }
      }
    }
    if (tb + TILE > t1) {  // keys past this workgroup's range: no score, no value scale
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = tb + 16 * (e >> 2) + 4 * (e & 3) + q4;
        s[e] = tok < t1 ? s[e] : -INFINITY;
        vsc[e] = tok < t1 ? vsc[e] : 0.0f;
      }
    }
    // Lazy rescaling: p = 2^(csm s - m_run) with a running max that only moves when a score
    // exceeds it by more than LAZY_LOG2 (p <= 2^LAZY_LOG2 otherwise), so the cross-lane max and
    // the accumulator rescale leave the common path. The first tile always takes the update.
    float lm = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) lm = fmaxf(lm, s[e]);
    lm *= csm;
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
    for (int e = 0; e < 8; ++e) {
      s[e] = __builtin_amdgcn_exp2f(fmaf(s[e], csm, -m_use));
      psum += s[e];
    }
    l_run += psum;

    __builtin_amdgcn_s_setprio(1);
    // P' = p * vscale, split into bf16 hi + lo
    u32x4_t bhi, blo;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float a0 = s[2 * u] * vsc[2 * u];
      const float a1 = s[2 * u + 1] * vsc[2 * u + 1];
      const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a0, a1}, bf16x2_t));
      const float r0 = a0 - __builtin_bit_cast(float, h << 16);
      const float r1 = a1 - __builtin_bit_cast(float, h & 0xffff0000u);
      bhi[u] = h;
      blo[u] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t));
    }
    // hi products of four dims-sets, then their lo products, so that the two MFMAs into one
    // accumulator are separated by three independent ones
#pragma unroll
    for (int k0 = 0; k0 < 8; k0 += 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[k0 + j] = mfma_bf16(va[k0 + j], bhi, acc[k0 + j]);
      if (k0 == 0) corr = mfma_bf16(ones, bhi, corr);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[k0 + j] = mfma_bf16(va[k0 + j], blo, acc[k0 + j]);
      if (k0 == 4) corr = mfma_bf16(ones, blo, corr);
    }
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_wave_barrier();
  };

  // 3-deep ring of LDS tiles: the loads of the next 2 tiles are in flight while one is processed
  // (unrolled by 3 so that each ring position is its own LDS object; a 4th buffer, the whole
  // 160 KB of LDS per CU at 2 workgroups, measured no faster)
  for (int i = 0; i < nw; i += 3) {
    if (i + 2 < nw) issue_tile<G, MASK>(R, tile_key(i + 2), S, tiles2[wave], lane);
    process(i, tiles0[wave]);
    if (i + 1 >= nw) break;
    if (i + 3 < nw) issue_tile<G, MASK>(R, tile_key(i + 3), S, tiles0[wave], lane);
    process(i + 1, tiles1[wave]);
    if (i + 2 >= nw) break;
    if (i + 4 < nw) issue_tile<G, MASK>(R, tile_key(i + 4), S, tiles1[wave], lane);
    process(i + 2, tiles2[wave]);
  }

  // per-wave partial -> LDS (in the wave's first tile buffer, whose last reads are complete)
  // wave w's partial: o [NREP][FAST_D], then m [NREP] and l [NREP]
  auto o_wave = [&](int w) -> float* {
    if constexpr (O_IN_TILE) return (float*)&tiles0[w];
    else return &o_sep[w * (NREP * FAST_D + 2 * NREP)];
  };
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  const bool own = colvalid && (q4 / CPG == colm);
  float* ow = o_wave(wave);
  if (own) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ow[colh * FAST_D + 32 * q4 + 8 * r + k] = acc[k][r] - 24.0f * corr[r];
      }
    }
  }
  if (lane < NREP) {
    ow[NREP * FAST_D + lane] = m_run;
    ow[NREP * FAST_D + NREP + lane] = l_run;
  }
  __syncthreads();

  // merge the 4 waves
  for (int idx = tid; idx < NREP * FAST_D; idx += THREADS) {
    const int h = idx / FAST_D;
    const int d = idx - h * FAST_D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, o_wave(w)[NREP * FAST_D + h]);
    float L = 0.0f;
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float mw = o_wave(w)[NREP * FAST_D + h];
      const float wt = (mw == -INFINITY) ? 0.0f : exp2f(mw - M);
      L += wt * o_wave(w)[NREP * FAST_D + NREP + h];
      a += wt * o_wave(w)[h * FAST_D + d];
    }
    const int qh = kvh * NREP + h;
    if (p.nsplit == 1) {
      store_float(p.out.data, p.out.dtype, b * p.out.s[0] + qh * p.out.s[1] + d * p.out.s[2],
                  a / L);
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + qh) * p.nsplit + split;
      coherent_store(&p.ws_acc[slot * FAST_D + d], a);
      if (d == 0) {
        coherent_store(&p.ws_m[slot], M);
        coherent_store(&p.ws_l[slot], L);
      }
    }
  }
  if (p.nsplit > 1 && p.fold) {
    // Folded split-K merge: the last of the unit's nsplit workgroups to arrive merges all of
    // them and puts the unit's counter back to 0, so a call leaves every counter as it found it.
    // No workgroup waits for another. The partials go through device-coherent accesses (written
    // through past this XCD's L2, read past the merging XCD's), and each thread's stores have
    // completed (vmcnt counts stores on gfx9) before the workgroup's arrival is counted, so the
    // last arrival sees every split's partials. A device-scope fence instead (__threadfence:
    // a write-back and an invalidate of the whole L2 per workgroup) made batch 1, ctx 4096 take
    // 32.4 instead of 14.0 us.
    __shared__ int s_last;
    __shared__ float s_w[FOLD_MAX_PARTIALS], s_wl[FOLD_MAX_PARTIALS], s_L[16];
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      s_last = __hip_atomic_fetch_add(&p.ws_cnt[unit], 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(p.nsplit - 1);
    }
    __syncthreads();
    if (!s_last) return;
    merge_unit<NREP>(p, b, kvh, s_w, s_wl, s_L);
    if (tid == 0) __hip_atomic_store(&p.ws_cnt[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

bool fast_fold_fits(int nrep, int nsplit) {
  return (int64_t)nrep * nsplit <= FOLD_MAX_PARTIALS;
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

bool fast_path_ok(const AttnParams& p) {
  if (diag(LQ_DIAG_ATTN_FORCE_GENERIC)) return false;
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
  // the mask row loads per lane with a 32-bit key stride and a 32-bit extent
  if (p.mask != nullptr) {
    if (p.mask_sk <= 0 || ((uintptr_t)p.mask & 3) != 0) return false;
    if (p.mask_len * p.mask_sk * 4 >= ((int64_t)1 << 31)) return false;
  }
  return true;
}

// CUs of the current device and the workgroups per CU that the occupancy calculator gives for
// the <4, 4> instance of attn_fast_kernel (its register and LDS use stand for the others').
struct FastResidency {
  int cus, per_cu;
};

static FastResidency fast_residency() {
  static FastResidency cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FastResidency{256, 2};
  if (cached[dev].cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&attn_fast_kernel<4, 4, false>), THREADS, 0) != hipSuccess ||
        per_cu <= 0) {
      per_cu = 2;
    }
    cached[dev] = FastResidency{cus, per_cu};
  }
  return cached[dev];
}

SplitPlan plan_fast(int64_t B, int64_t Hkv, int64_t S) {
  // One resident generation of waves: each wave gets as many keys as that takes (rounded to the
  // 32-key tile, 4 waves per workgroup split, the split's tiles dealt to the waves in turn).
  // Fewer, longer waves amortize the per-wave setup and the 4-wave merge, and at
  // B * Hkv >= resident / 4 no split-K merge runs at all.
  const FastResidency r = fast_residency();
  const int64_t target_waves = (int64_t)r.cus * r.per_cu * WAVES;
  int64_t tpw = (B * Hkv * S + target_waves - 1) / target_waves;
  tpw = ((tpw + TILE - 1) / TILE) * TILE;
  tpw = std::min<int64_t>(std::max<int64_t>(tpw, TILE), (int64_t)1 << 20);
  // A wave of one or two tiles spends most of its time in set-up and the merges, so a wave takes
  // at least 4 tiles while that still leaves a workgroup for every CU (batch 1, ctx 16384: 32
  // splits instead of 64, 17.8 against 20.0 us; at ctx 1024 and 4096 4 tiles would leave 16 and
  // 64 workgroups and ran slower, 15.8 and 16.8 against 13.7 and 14.2 us).
  constexpr int64_t kMinTiles = 4 * TILE;
  if (tpw < kMinTiles && B * Hkv * ((S + WAVES * kMinTiles - 1) / (WAVES * kMinTiles)) >= r.cus) {
    tpw = kMinTiles;
  }
  SplitPlan sp{};
  sp.chunk = WAVES * tpw;
  sp.nsplit = (int)std::max<int64_t>(1, (S + sp.chunk - 1) / sp.chunk);
  return sp;
}

template <int NREP, int G>
static void launch_one(const AttnParams& p, hipStream_t st) {
  const dim3 grid((unsigned)(p.B * p.Hkv), (unsigned)p.nsplit);
  if (p.mask != nullptr) {
    hipLaunchKernelGGL((attn_fast_kernel<NREP, G, true>), grid, dim3(THREADS), 0, st, p);
  } else {
    hipLaunchKernelGGL((attn_fast_kernel<NREP, G, false>), grid, dim3(THREADS), 0, st, p);
  }
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
