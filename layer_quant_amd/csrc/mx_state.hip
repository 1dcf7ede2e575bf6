// MX8 / MX4 Mamba2 recurrent state: fused selective-state update, block encoder, decoder.
//
// Replaces the reference's Triton kernels in hybrid_quant/mamba_state_8b_kernel.py:
//   _state_update_requant_mx8_row_kernel (:33-222)              -> mx_update_kernel<8, .>
//   _state_update_mx8_kernel + _requantize_mx4_kernel (:225-544) -> mx_update_kernel<4, .>
//   _quantize_initial_state_mx (:547-572, torch)                 -> mx_encode_kernel<., RNE>
//
// Layout (reference MambaStateKernelCache, :19-25), per state row (b, h, p) of N values:
//   q_state    int8  [N]     one byte per mantissa in both formats
//   shared_exp uint8 [N/16]  biased exponent of each 16-value block (127 = 2^0)
//   micro_exp  uint8 [N/2]   0/1 per pair of values
// One lane owns one 16-value block: a 16-byte mantissa load, an 8-byte micro-exponent load and a
// 1-byte exponent load, all coalesced across the wave; the row's N/16 lanes are adjacent, so
// y = sum_n h'_n C_n is a shuffle reduction inside the row's lane group. The update is one pass:
// the MX4 path does not round-trip an fp32 state through HBM as the reference does.
//
// Encode of a block (bit-exact with the torch formula):
//   t = max(absmax / (2M), 1e-30)           correctly rounded fp32 quotient (two fmas)
//   e = clamp(ceil(log2 t) + 127, 1, 254)    ceil of the correctly rounded fp32 log2, computed
//                                            exactly from t's exponent and mantissa bits
//   base = absmax == 0 ? 1 : 2^(e-127);  micro = pair_absmax > M*base
//   qa = min(|v| / (base*2^micro), M)        as a product with the exact reciprocal
//   level = rint(qa) | floor(qa + 0.5) | floor(qa) + (u < qa - floor(qa))   (always <= M)
// The counter mode (LQ_ROUND_SR_COUNTER) draws 16-bit integers u16 and dithers on a 2^-16 grid:
//   t = RN(v / (base*2^micro) + 192 + u16 * 2^-16)  (one fma),  level = floor(t) - 192
// The Philox mode (LQ_ROUND_SR_PHILOX) draws the reference's own u = tl.rand(seed, offset) per
// element (Philox4x32-10, philox_uniform below) and applies the supplied-uniform formula.
#include <math.h>
#include <stdlib.h>

#include <type_traits>

#include "lq_common.h"
#include "state_common.h"

namespace lq {

struct MxState {
  int8_t* q;
  uint8_t* e;
  uint8_t* mi;
  int64_t qs[3], es[3], ms[3];  // strides of (b, h, p); the innermost dimension is contiguous
};

struct MxUpdateParams {
  MxState st;
  View x, dt, dtb, A, B, C, D, z, out, uni;
  int Bn, H, P, N, ratio, bpr, vbpr_log2;
  int has_dtb, has_D, has_z, softplus, a_row_const;
  uint32_t key;
  uint32_t pk0, pk1;  // Philox mode: the key words lo32(seed), hi32(seed)
  uint64_t rng_offset;
  // counter and Philox modes: an optional step on the device (int64 [1]) and its stride B*H*P*N; the counter
  // offset is rng_offset + step * stride (the reference's step*B*H*P*N, the step read by the
  // kernel, so that a captured graph advancing it between replays draws anew on every replay)
  const int64_t* step_dev;
  uint64_t step_stride;
  // rows kernel, counter mode without a device step: the counter base (below), from the host
  uint32_t kh, kh1, lo_base;
  // rows kernel: byte stride between rows of x, z and out, and the byte span of one
  // (batch, head) slice of each rounded up to 4 (0 for an absent z)
  uint32_t x_row_bytes, z_row_bytes, out_row_bytes;
  uint32_t x_span, z_span, out_span;
  // rows kernel, supplied-uniform mode: byte stride between rows of the uniform tensor and the
  // byte span of one (batch, head) slice of it
  uint32_t uni_row_bytes, uni_span;
};

struct MxCodecParams {
  MxState st;
  View v;    // float state [B, H, P, N] (encode input or decode output)
  View uni;  // uniforms for LQ_ROUND_SR_UNIFORM
  int Bn, H, P, N, bpr, vbpr_log2;
  uint32_t key;
  uint32_t pk0, pk1;  // Philox mode: the key words lo32(seed), hi32(seed)
  uint64_t rng_offset;
};

// State layouts: the reference's (one byte per mantissa, one byte per pair micro-exponent), and
// the compact ones (micro-exponents as bits, bit k of byte j = pair 8j + k of the row; MX4
// mantissas as two's-complement nibbles, byte p = value 2p in the low nibble, 2p + 1 in the high).
// The exponent bytes are the reference's in all three.
enum { LAYOUT_REF = 0, LAYOUT_CM8 = 1, LAYOUT_CM4 = 2 };
template <int LY>
struct LayoutOf {
  static constexpr bool qnib = LY == LAYOUT_CM4;   // nibble mantissas
  static constexpr bool mbits = LY != LAYOUT_REF;  // bit micro-exponents
  static constexpr int qbytes = qnib ? 8 : 16;     // mantissa bytes per 16-value block
  static constexpr int mbytes = mbits ? 1 : 8;     // micro-exponent bytes per block
};

// Mantissa n of a block's raw words, as float.
template <int LY>
__device__ __forceinline__ float mant(const uint32_t (&qw)[4], int n) {
  if constexpr (LayoutOf<LY>::qnib) {
    // the builtin's result type is unsigned: the signed field must be converted as an int
    return (float)(int)__builtin_amdgcn_sbfe(qw[n >> 3], 4 * (n & 7), 4);
  } else {
    return (float)(int)(int8_t)(qw[n >> 2] >> (8 * (n & 3)));
  }
}

// Micro-exponent of pair k of a block (the reference layout keeps the whole byte: e + micro
// forms the scale exponent there).
template <int LY>
__device__ __forceinline__ uint32_t micro(const uint32_t (&mw)[2], int k) {
  if constexpr (LayoutOf<LY>::mbits) {
    return (mw[0] >> k) & 1u;
  } else {
    return (mw[k >> 2] >> (8 * (k & 3))) & 0xffu;
  }
}

// A constant held in an SGPR: a select between 0 and it is one v_cndmask_b32 (the compiler
// otherwise materialises each shifted flag constant in a VGPR with a v_mov first).
__device__ __forceinline__ uint32_t sgpr_const(uint32_t c) {
  uint32_t r;
  asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(c));
  return r;
}

// Level bytes qw[4] (one int8 per value) and micro flags mi[8] of an encoded block, in the
// layout's raw form: nibbles qw[0..1] and micro bits mw[0] for the compact layouts.
template <int LY>
__device__ __forceinline__ void pack_block(uint32_t (&qw)[4], uint32_t (&mw)[2],
                                           const bool (&mi)[8]) {
  if constexpr (LayoutOf<LY>::qnib) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t ev = __builtin_amdgcn_perm(qw[2 * w + 1], qw[2 * w], 0x06040200u);
      const uint32_t od = __builtin_amdgcn_perm(qw[2 * w + 1], qw[2 * w], 0x07050301u);
      qw[w] = (ev & 0x0f0f0f0fu) | ((od << 4) & 0xf0f0f0f0u);
    }
    qw[2] = 0;
    qw[3] = 0;
  }
  if constexpr (LayoutOf<LY>::mbits) {
    uint32_t bits = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) bits |= mi[k] ? (k == 7 ? sgpr_const(0x80u) : 1u << k) : 0u;
    mw[0] = bits;
    mw[1] = 0;
  } else {
    const uint32_t b1 = sgpr_const(0x100u), b2 = sgpr_const(0x10000u), b3 = sgpr_const(0x1000000u);
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      mw[w] = (mi[4 * w] ? 1u : 0u) | (mi[4 * w + 1] ? b1 : 0u) | (mi[4 * w + 2] ? b2 : 0u) |
              (mi[4 * w + 3] ? b3 : 0u);
    }
  }
}

// lowbias32 without its last step (x ^= x >> 16): the counter mode's word formation below
// performs that step while it makes the draws' offsets.
__device__ __forceinline__ uint32_t lowbias32_pre(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  return x;
}
__device__ __forceinline__ uint32_t lowbias32(uint32_t x) {
  x = lowbias32_pre(x);
  return x ^ (x >> 16);
}

// The two dither offsets of one hash word from x = lowbias32_pre(...): with W = x ^ (x >> 16)
// (lowbias32's output), th = bits of 192 + (W >> 16) * 2^-16 and tl = bits of
// 192 + (W & 0xffff) * 2^-16. th is one v_perm_b32 (x's high half under 0x4340, the bits of
// 192.0), and tl one v_bitop3_b32 (x ^ th in the low half, th's 0x4340 in the high half): two
// instructions where the shift, mask, xor and two ors took four.
__device__ __forceinline__ void dither_words(uint32_t x, uint32_t& tl, uint32_t& th) {
  th = __builtin_amdgcn_perm(sgpr_const(0x43400000u), x, 0x07060302u);
  tl = ((x ^ th) & 0x0000ffffu) | (th & 0xffff0000u);
}

// Triton's tl.rand(seed, c) for the 64-bit offset c (triton/language/random.py, the stream of the
// reference's writeback, hybrid_quant/mamba_state_8b_kernel.py:198, 405, 479, 529): Philox4x32
// with 10 rounds (Salmon et al., SC'11) of the counter (lo32(c), hi32(c), 0, 0) under the key
// (lo32(seed), hi32(seed)); its first word x, as int32, becomes (x < 0 ? -x - 1 : x) * 0x1.fffffep-32
// in fp32. The key schedule is the same for every lane (scalar registers).
__device__ __forceinline__ float philox_uniform(uint32_t k0, uint32_t k1, uint64_t c) {
  constexpr uint32_t RA = 0xD2511F53u, RB = 0xCD9E8D57u, KA = 0x9E3779B9u, KB = 0xBB67AE85u;
  uint32_t c0 = (uint32_t)c, c1 = (uint32_t)(c >> 32), c2 = 0u, c3 = 0u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    // one 32 x 32 -> 64-bit product per multiplier (v_mad_u64_u32 gives both halves at the cost
    // of one v_mul_hi_u32) and one three-way xor (v_bitop3_b32, full rate) per word
    const uint64_t pa = (uint64_t)RA * c0, pb = (uint64_t)RB * c2;
    c0 = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c1, k0, 0x96);
    c2 = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c3, k1, 0x96);
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    k0 += KA;
    k1 += KB;
  }
  const int32_t x = (int32_t)c0;
  return (float)(x < 0 ? ~x : x) * 0x1.fffffep-32f;
}

// The Philox draws of one 16-value block (element i at offset c0 + i) scaled by 2^16 (exact),
// in the form encode16 takes supplied uniforms.
__device__ __forceinline__ void philox_block_u16(uint32_t k0, uint32_t k1, uint64_t c0,
                                                 float (&u16)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) u16[i] = philox_uniform(k0, k1, c0 + (uint64_t)i) * 65536.0f;
}

// Counter offset of an update: rng_offset plus, when the step lives on the device, step * stride.
__device__ __forceinline__ uint64_t counter_offset(const MxUpdateParams& p) {
  return p.step_dev == nullptr ? p.rng_offset
                               : p.rng_offset + (uint64_t)(*p.step_dev) * p.step_stride;
}

// The row kernel's counter base: the low word of offset / 2 (the first pair counter) and the
// hashes K_hi = lowbias32(hi ^ key) of its high word hi and of hi + 1 (a launch's pair counters
// span fewer than 2^31 values, so they cross at most one high-word boundary).
struct CounterBase {
  uint32_t lo_base, kh, kh1;
};

__device__ __forceinline__ CounterBase counter_base(const MxUpdateParams& p) {
  if (p.step_dev == nullptr) return CounterBase{p.lo_base, p.kh, p.kh1};
  const uint64_t pair0 = counter_offset(p) >> 1;
  const uint32_t hi = (uint32_t)(pair0 >> 32);
  return CounterBase{(uint32_t)pair0, lowbias32(hi ^ p.key), lowbias32((hi + 1u) ^ p.key)};
}

// ceil(log2(t)) with log2 correctly rounded to fp32, for positive normal t (or +inf).
// t = 2^E * (1 + j 2^-23): the result is E if j == 0 or if E + log2(1 + j 2^-23) rounds back to
// E in fp32, which happens for 0 < j <= T; T = floor(2^(kk-1) ln 2) where 2^(kk-24) is half the
// fp32 spacing at E (kk = floor(log2|E|), one less for negative powers of two; E = 0 -> T = 0).
__device__ __forceinline__ int ceil_log2_exact(float t) {
  const uint32_t bits = __float_as_uint(t);
  const int E = (int)((bits >> 23) & 0xffu) - 127;
  const uint32_t mant = bits & 0x7fffffu;
  const int a = E < 0 ? -E : E;
  const int am = a > 0 ? a : 1;
  const int fl = 31 - __clz(am);
  const bool pow2 = (am & (am - 1)) == 0;
  const int kk = (E < 0 && pow2) ? fl - 1 : fl;
  const uint32_t thr = (E == 0) ? 0u : (uint32_t)ldexpf(0.693147182f, kk - 1);
  return mant == 0 ? E : (mant <= thr ? E : E + 1);
}

// Counter-based draws of one 16-value block: element n draws counter c = rng_offset + row*N + n;
// pair c>>1 hashes to the 32-bit word W = lowbias32(...) (k = pair within the block), whose low
// half is the even element's 16-bit draw and whose high half is the odd element's; pw[k] holds
// lowbias32_pre's value, which dither_words turns into both draws' offsets.
__device__ __forceinline__ void block_words(uint32_t key, uint64_t c0, uint32_t (&pw)[8]) {
  const uint64_t pc0 = c0 >> 1;
  const uint32_t lo0 = (uint32_t)pc0;
  const uint32_t hi0 = (uint32_t)(pc0 >> 32);
  const uint32_t kh0 = lowbias32(hi0 ^ key);
  uint32_t kh[8];
  if (__builtin_expect(lo0 > 0xfffffff8u, 0)) {  // the low word wraps inside this block
    const uint32_t kh1 = lowbias32((hi0 + 1u) ^ key);
#pragma unroll
    for (int k = 0; k < 8; ++k) kh[k] = (lo0 + (uint32_t)k < lo0) ? kh1 : kh0;
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) kh[k] = kh0;
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) pw[k] = lowbias32_pre((lo0 + (uint32_t)k) ^ kh[k]);
}

// Shared exponent of a block from its absmax: eb = clamp(ceil(log2 t) + 127, 1, 254) with
// t = max(RN(absmax / 2M), 1e-30), and ebase = 127 for an all-zero block. RN(a / 2M) is
// q + (a - 2M q) / 2M evaluated as q = RN(a c), r = fma(-q, 2M, a) (exact), RN(fma(r, c, q)) with
// c = RN(1 / 2M); that equals the IEEE quotient for every positive fp32 a once the 1e-30 floor
// is applied (checked exhaustively for 2M = 14 and 126; +inf is passed through).
// ceil(log2 t) is E + 1 unless t lies within T(E) <= 44 ulps above 2^E (T = 0 for E = 0), where
// the exact rule decides. Returns whether it did: only then (t within the band, or +inf) can
// 2^e fall below absmax / 2M, so that |v| / (base * 2^micro) may exceed M. Elsewhere e = E + 1
// and absmax / 2M <= t (1 + 2^-24) < 2^(E+1) (the eb clamp only raises the scale), so every
// pair's qa <= M exactly.
template <int FB>
__device__ __forceinline__ bool block_exponent(float amax, int& eb, int& ebase) {
#pragma clang fp contract(off)
  constexpr float TWO_M = FB == 8 ? 126.0f : 14.0f;
  constexpr float C = 1.0f / TWO_M;
  const float q = amax * C;
  const float r = __builtin_fmaf(-q, TWO_M, amax);
  float t = __builtin_fmaf(r, C, q);
  t = (amax == INFINITY) ? amax : t;
  t = fmaxf(t, 1.0e-30f);
  const uint32_t bits = __float_as_uint(t);
  int e = (int)(bits >> 23) - 126;
  const bool band = (bits & 0x7fffffu) <= 44u;
  if (band) e = ceil_log2_exact(t);
  eb = min(max(e + 127, 1), 254);
  ebase = (amax == 0.0f) ? 127 : eb;
  return band;
}

// block_exponent with a fast path. For absmax in [2^-92, 2^120), q = RN(absmax * RN(1/2M)) lies
// within 2 ulps of t = RN(absmax / 2M) (q = (absmax/2M)(1 + d)(1 + f), |d|, |f| <= 2^-24); when
// q's mantissa field is in [48, 2^23 - 4], t is in q's binade, more than 44 ulps above its power
// of two, and t > 1e-30, so eb = E(q) + 128 with no clamp (eb in [29, 245]) and no band. Other
// blocks take the exact rule. (Checked against block_exponent for every positive fp32 absmax.)
constexpr uint32_t FAST_AMAX_LO = 0x11800000u;  // 2^-92
constexpr uint32_t FAST_AMAX_HI = 0x7b800000u;  // 2^120
constexpr uint32_t FAST_MANT_LO = 48u;
constexpr uint32_t FAST_MANT_HI = 0x7ffffcu;

template <int FB>
__device__ __forceinline__ bool block_exponent_fast(float amax, int& eb, int& ebase) {
  constexpr float C = FB == 8 ? 1.0f / 126.0f : 1.0f / 14.0f;
  const uint32_t qb = __float_as_uint(amax * C);
  const bool fast = (__float_as_uint(amax) - FAST_AMAX_LO) < (FAST_AMAX_HI - FAST_AMAX_LO) &&
                    ((qb & 0x7fffffu) - FAST_MANT_LO) <= (FAST_MANT_HI - FAST_MANT_LO);
  if (__builtin_expect(fast, 1)) {
    eb = (int)(qb >> 23) + 1;
    ebase = eb;
    return false;
  }
  return block_exponent<FB>(amax, eb, ebase);
}

// max(|a|, |b|) and max(a, b, c) as single instructions: the operands are arithmetic results
// (never signalling NaNs), so the canonicalising moves the compiler adds for fmaxf are not needed.
__device__ __forceinline__ float abs_max2(float a, float b) {
  float r;
  asm("v_max_f32_e64 %0, |%1|, |%2|" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max_with_zero(float a, float b) {
  float r;
  asm("v_max3_f32 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// t + (w & 0xffff) and t + (w >> 16) as single SDWA adds.
__device__ __forceinline__ int add_word0(int t, uint32_t w) {
  int r;
  asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
      : "=v"(r) : "v"(t), "v"(w));
  return r;
}
__device__ __forceinline__ int add_word1(int t, uint32_t w) {
  int r;
  asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
      : "=v"(r) : "v"(t), "v"(w));
  return r;
}

// Keeps a value opaque to the optimiser, so that two precomputed alternatives stay two registers
// and a select between them is not rewritten into a select of their inputs.
template <typename T>
__device__ __forceinline__ T pin(T v) {
  asm("" : "+v"(v));
  return v;
}

// Pair maxima and the block absmax of 16 values, max(0, |v_0|, ..., |v_15|) with NaNs ignored
// (IEEE maxNum), as a running fmaxf from 0 gives.
__device__ __forceinline__ float pair_maxima(const float (&v)[16], float (&pa)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) pa[k] = abs_max2(v[2 * k], v[2 * k + 1]);
  const float m = max3(max3(pa[0], pa[1], pa[2]), pa[3], pa[4]);
  return max_with_zero(max3(m, pa[5], pa[6]), pa[7]);
}

// Exact reciprocal of the pair scale 2^(se-127): normal for se <= 253, the subnormal 2^-127 for
// se = 254, and 0 for se = 255 (scale +inf; only reachable when absmax is +inf, as |v| / inf is 0).
__device__ __forceinline__ float pair_recip(int se) {
  return se <= 253 ? __uint_as_float((uint32_t)(254 - se) << 23)
                   : (se == 254 ? __uint_as_float(0x00400000u) : 0.0f);
}

// Encode 16 values in the nearest-even, half-up or supplied-uniform mode. `u16` holds the
// supplied uniforms scaled by 2^16 (so that the comparison u < frac becomes u16 < frac * 2^16,
// both sides exact), unused otherwise. The reference's final min(level, M) is omitted: every mode
// already yields level <= M.
template <int FB, int RMODE, int LY>
__device__ __forceinline__ void encode16(const float (&v)[16], const float (&u16)[16],
                                         uint32_t (&qw)[4], uint32_t (&mw)[2], uint32_t& eb_out) {
#pragma clang fp contract(off)
  constexpr float M = FB == 8 ? 63.0f : 7.0f;
  float pa[8];
  const float amax = pair_maxima(v, pa);
  int eb, ebase;
  block_exponent_fast<FB>(amax, eb, ebase);
  const float thr = M * __uint_as_float((uint32_t)ebase << 23);
  // exact reciprocals of the pair scales 2^(se-127), se = ebase + micro
  const float inv0 = pair_recip(ebase);
  const float inv1 = pair_recip(ebase + 1);
  int qi[16];
  bool mb[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const bool mi = pa[k] > thr;
    const float inv = mi ? inv1 : inv0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float qa = fminf(fabsf(v[2 * k + i]) * inv, M);
      float lvl;
      if constexpr (RMODE == LQ_ROUND_NEAREST_EVEN) {
        lvl = rintf(qa);
      } else if constexpr (RMODE == LQ_ROUND_HALF_UP) {
        lvl = floorf(qa + 0.5f);
      } else {
        const float fl = floorf(qa);
        lvl = fl + ((u16[2 * k + i] < (qa - fl) * 65536.0f) ? 1.0f : 0.0f);
      }
      // sign of v (v < 0 -> negative level; -0.0 gives level 0 either way)
      qi[2 * k + i] = (int)copysignf(lvl, v[2 * k + i]);
    }
    mb[k] = mi;
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)qi[4 * w + 1], (uint32_t)qi[4 * w], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)qi[4 * w + 3], (uint32_t)qi[4 * w + 2], 0x04000c0cu);
    qw[w] = lo | hi;
  }
  pack_block<LY>(qw, mw, mb);
  eb_out = (uint32_t)eb;
}

// Encode 16 values in the counter mode. With q = v / pair_scale (signed) and the element's 16-bit
// draw u16, t = RN(q + 192 + u16 * 2^-16) is one fma: v times the exact reciprocal of the pair
// scale, plus 192 + u16 * 2^-16 made from the draw's bits (0x43400000 | u16). t lies in
// [129, 256), where the fp32 spacing is exactly 2^-16, so byte 2 of its bits is
// floor(t) - 128 = level + 64, level = floor(RN_{2^-16}(q + u16 * 2^-16)) in [-M, M]; a carry-free
// byte fix turns level + 64 into the int8 level. Blocks whose exponent came from the exact rule
// (see block_exponent), where |q| may exceed M, clamp t to [192 - M, 193 + M - 2^-16]: the same
// levels as clamping q to [-M, M] first (floor(M + u) = M, floor(-M + u) = -M).
// word(k) returns lowbias32_pre's value x for pair k (with W = x ^ (x >> 16), the low half of W
// is the even element's draw and the high half the odd element's). Each word is made just before its two fmas use it, and the next word
// waits for them: computed all at once, the eight words and the block's values were live
// together (91 VGPRs in the reference layout's row kernel instead of 77).
template <int FB, int LY, class WordFn>
__device__ __forceinline__ void encode16_dither(const float (&v)[16], WordFn&& word,
                                                uint32_t (&qw)[4], uint32_t (&mw)[2],
                                                uint32_t& eb_out) {
#pragma clang fp contract(off)
  constexpr float M = FB == 8 ? 63.0f : 7.0f;
  float pa[8];
  const float amax = pair_maxima(v, pa);
  int eb, ebase;
  const bool band = block_exponent_fast<FB>(amax, eb, ebase);
  const float thr = M * __uint_as_float((uint32_t)ebase << 23);
  // pair_recip(ebase) and pair_recip(ebase + 1) without branches (ebase <= 254)
  const float inv0 = pin(ebase <= 253 ? __uint_as_float((uint32_t)(254 - ebase) << 23)
                                      : __uint_as_float(0x00400000u));
  const float inv1 = pin(ebase <= 253 ? inv0 * 0.5f : 0.0f);
  float t[16];
  bool mb[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const bool mi = pa[k] > thr;
    const float inv = mi ? inv1 : inv0;
    uint32_t tl, th;
    dither_words(word(k), tl, th);
    t[2 * k] = __builtin_fmaf(v[2 * k], inv, __uint_as_float(tl));
    t[2 * k + 1] = __builtin_fmaf(v[2 * k + 1], inv, __uint_as_float(th));
    word.after(t[2 * k], t[2 * k + 1]);
    mb[k] = mi;
  }
  if (band) {  // rare
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      t[i] = __builtin_amdgcn_fmed3f(t[i], 192.0f - M, 193.0f + M - 0x1p-16f);
    }
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(t[4 * w + 1]),
                                              __float_as_uint(t[4 * w]), 0x0c0c0602u);
    const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(t[4 * w + 3]),
                                              __float_as_uint(t[4 * w + 2]), 0x06020c0cu);
    // bytes b = level + 64 in [1, 127] -> (b - 64) mod 256 = (b + 64) ^ 128, where b + 64 <= 191
    // stays inside its byte (lo and hi hold disjoint bytes, so their sum is their union: one
    // v_add3_u32, which the compiler would split into an or and an add)
    uint32_t b;
    asm("v_add3_u32 %0, %1, %2, %3" : "=v"(b) : "v"(lo), "v"(hi), "s"(sgpr_const(0x40404040u)));
    qw[w] = b ^ 0x80808080u;
  }
  pack_block<LY>(qw, mw, mb);
  eb_out = (uint32_t)eb;
}

// Hash words of a block for encode16_dither: from a precomputed array (the general kernel), or
// hashed on demand from the block's pair-counter base (the row kernel: base = (lo32 of the first
// pair counter) ^ K_hi after lowbias32's first xorshift, the block's pairs differing only in the
// low 3 bits). after() makes the next word wait for the previous pair's fmas.
struct ArrayWords {
  const uint32_t (&pw)[8];
  __device__ __forceinline__ uint32_t operator()(int k) const { return pw[k]; }
  __device__ __forceinline__ void after(float, float) const {}
};

struct HashWords {
  uint32_t base;
  __device__ __forceinline__ uint32_t operator()(int k) const {
    uint32_t x = base ^ (uint32_t)k;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    return x;  // lowbias32_pre's value: dither_words does the last step
  }
  __device__ __forceinline__ void after(float a, float b) {
    asm volatile("" : "+v"(base) : "v"(a), "v"(b));
  }
};

// Raw words of one block at q / mi / e (VEC: q and mi aligned to their block size).
template <bool VEC, int LY>
__device__ __forceinline__ void load_block(const int8_t* q, const uint8_t* mi, const uint8_t* e,
                                           uint32_t (&qw)[4], uint32_t (&mw)[2], uint32_t& ev) {
  using L = LayoutOf<LY>;
  const uint8_t* qb = (const uint8_t*)q;
  qw[2] = qw[3] = 0;
  mw[1] = 0;
  if constexpr (VEC && L::qbytes == 16) {
    const uint4 a = *(const uint4*)q;
    qw[0] = a.x;
    qw[1] = a.y;
    qw[2] = a.z;
    qw[3] = a.w;
  } else if constexpr (VEC) {
    const uint2 a = *(const uint2*)q;
    qw[0] = a.x;
    qw[1] = a.y;
  } else {
#pragma unroll
    for (int w = 0; w < L::qbytes / 4; ++w) {
      qw[w] = qb[4 * w] | (qb[4 * w + 1] << 8) | (qb[4 * w + 2] << 16) | ((uint32_t)qb[4 * w + 3] << 24);
    }
  }
  if constexpr (L::mbits) {
    mw[0] = *mi;
  } else if constexpr (VEC) {
    const uint2 m = *(const uint2*)mi;
    mw[0] = m.x;
    mw[1] = m.y;
  } else {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      mw[w] = mi[4 * w] | (mi[4 * w + 1] << 8) | (mi[4 * w + 2] << 16) | ((uint32_t)mi[4 * w + 3] << 24);
    }
  }
  ev = *e;
}

template <bool VEC, int LY>
__device__ __forceinline__ void store_block(int8_t* q, uint8_t* mi, uint8_t* e,
                                            const uint32_t (&qw)[4], const uint32_t (&mw)[2],
                                            uint32_t ev) {
  using L = LayoutOf<LY>;
  uint8_t* qb = (uint8_t*)q;
  if constexpr (VEC && L::qbytes == 16) {
    *(uint4*)q = make_uint4(qw[0], qw[1], qw[2], qw[3]);
  } else if constexpr (VEC) {
    *(uint2*)q = make_uint2(qw[0], qw[1]);
  } else {
#pragma unroll
    for (int i = 0; i < L::qbytes; ++i) qb[i] = (uint8_t)(qw[i >> 2] >> (8 * (i & 3)));
  }
  if constexpr (L::mbits) {
    *mi = (uint8_t)mw[0];
  } else if constexpr (VEC) {
    *(uint2*)mi = make_uint2(mw[0], mw[1]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) mi[i] = (uint8_t)(mw[i >> 2] >> (8 * (i & 3)));
  }
  *e = (uint8_t)ev;
}

// h_n = q_n * 2^(e - 127 + micro_pair(n)); the scale is built from exponent bits
// (e + micro = 255 gives +inf, as exp2(128) does in fp32).
template <int LY>
__device__ __forceinline__ void decode16(const uint32_t (&qw)[4], const uint32_t (&mw)[2],
                                         uint32_t ev, float (&h)[16]) {
  const uint32_t evs = ev << 23;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float sc = __uint_as_float((micro<LY>(mw, k) << 23) + evs);
#pragma unroll
    for (int i = 0; i < 2; ++i) h[2 * k + i] = mant<LY>(qw, 2 * k + i) * sc;
  }
}

// Supplied uniforms of one block (LQ_ROUND_SR_UNIFORM) scaled by 2^16; zeros otherwise.
template <int RMODE>
__device__ __forceinline__ void block_u16(const View& uni, int b, int h, int pp, int n0,
                                          float (&u16)[16]) {
  if constexpr (RMODE == LQ_ROUND_SR_UNIFORM) {
    const float* ub = (const float*)uni.data + ((int64_t)b * uni.s[0] + (int64_t)h * uni.s[1]);
    const int off = pp * (int)uni.s[2] + n0 * (int)uni.s[3];
#pragma unroll
    for (int i = 0; i < 16; ++i) u16[i] = ub[off + i * (int)uni.s[3]];
#pragma unroll
    for (int i = 0; i < 16; ++i) u16[i] *= 65536.0f;  // exact: u * 2^16
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) u16[i] = 0.0f;
  }
}

// Writeback encode of one block in mode RMODE; c0 = counter of the block's first element.
template <int FB, int RMODE, int LY>
__device__ __forceinline__ void encode_block(const float (&v)[16], const View& uni, uint32_t key,
                                             uint32_t pk0, uint32_t pk1, uint64_t c0, int b,
                                             int h, int pp, int n0, uint32_t (&qw)[4],
                                             uint32_t (&mw)[2], uint32_t& eb) {
  if constexpr (RMODE == LQ_ROUND_SR_COUNTER) {
    uint32_t pw[8];
    block_words(key, c0, pw);
    encode16_dither<FB, LY>(v, ArrayWords{pw}, qw, mw, eb);
  } else if constexpr (RMODE == LQ_ROUND_SR_PHILOX) {
    float u16[16];
    philox_block_u16(pk0, pk1, c0, u16);
    encode16<FB, LQ_ROUND_SR_UNIFORM, LY>(v, u16, qw, mw, eb);
  } else {
    float u16[16];
    block_u16<RMODE>(uni, b, h, pp, n0, u16);
    encode16<FB, RMODE, LY>(v, u16, qw, mw, eb);
  }
}

// Pointers to block blk of row pp of slice (b, h) in layout LY.
template <int LY>
__device__ __forceinline__ void block_ptrs(const MxState& st, int b, int h, int pp, int blk,
                                           int8_t*& qp, uint8_t*& mp, uint8_t*& ep) {
  using Lay = LayoutOf<LY>;
  qp = st.q + (int64_t)b * st.qs[0] + (int64_t)h * st.qs[1] + pp * (int)st.qs[2] + blk * Lay::qbytes;
  mp = st.mi + (int64_t)b * st.ms[0] + (int64_t)h * st.ms[1] + pp * (int)st.ms[2] + blk * Lay::mbytes;
  ep = st.e + (int64_t)b * st.es[0] + (int64_t)h * st.es[1] + pp * (int)st.es[2] + blk;
}

template <int FB, int RMODE, bool VEC, bool BCVEC, int LY>
__global__ __launch_bounds__(256) void mx_update_kernel(MxUpdateParams p) {
  const LaneIdx L = lane_index(p.P, p.vbpr_log2, p.bpr);
  const int b = L.b, h = L.h, pp = L.pp;
  const int n0 = L.blk * 16;

  int8_t* qp;
  uint8_t *mp, *ep;
  block_ptrs<LY>(p.st, b, h, pp, L.blk, qp, mp, ep);
  uint32_t qw[4], mw[2], ev;
  load_block<VEC, LY>(qp, mp, ep, qw, mw, ev);

  // per-row scalars (ms.py:134-139); exp and log use the hardware transcendentals (relative
  // error ~1e-6, far inside the 2e-3 output tolerance)
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
  const float dtx = dtv * xv;

  // h' = h * exp(A dt) + B dt x ; y = sum h' C (ms.py:158-159), h = q * 2^(e - 127 + micro)
  float hv[16];
  if (p.a_row_const) {
    // one decay per row: fold it into the power-of-two pair scale (exact), h' = fma(q, s*dA, .)
    const float dA = __expf(ldf(ab, p.A.dtype, aoff) * dtv);
    const uint32_t evs = ev << 23;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float sdA = __uint_as_float((micro<LY>(mw, k) << 23) + evs) * dA;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int n = 2 * k + i;
        hv[n] = fmaf(mant<LY>(qw, n), sdA, Bv[n] * dtx);
      }
    }
  } else {
    decode16<LY>(qw, mw, ev, hv);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float dA = __expf(ldf(ab, p.A.dtype, aoff + i * (int)p.A.s[2]) * dtv);
      hv[i] = fmaf(hv[i], dA, Bv[i] * dtx);
    }
  }
  float ypart = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ypart = fmaf(hv[i], Cv[i], ypart);
  if (!L.active) ypart = 0.0f;
  for (int o = (1 << p.vbpr_log2) >> 1; o > 0; o >>= 1) ypart += __shfl_xor(ypart, o, 64);
  if (L.in_range && L.blk == 0 && (threadIdx.x & ((1 << p.vbpr_log2) - 1)) == 0) {
    float y = ypart;
    if (p.has_D) y += xv * ldf(vbase(p.D, h, 0), p.D.dtype, pp * (int)p.D.s[1]);
    if (p.has_z) y *= ldf(vbase(p.z, b, h), p.z.dtype, pp * (int)p.z.s[2]);
    char* ob = (char*)vbase(p.out, b, h);
    const int oi = pp * (int)p.out.s[2];
    if (p.out.dtype == LQ_BF16) {
      ((uint16_t*)ob)[oi] = float_to_bf16_bits(y);
    } else if (p.out.dtype == LQ_F16) {
      ((_Float16*)ob)[oi] = (_Float16)y;
    } else {
      ((float*)ob)[oi] = y;
    }
  }

  // writeback encode (ms.py:168-222, 512-544)
  const uint64_t row = ((uint64_t)b * p.H + h) * p.P + pp;
  uint32_t eo_bits;
  encode_block<FB, RMODE, LY>(hv, p.uni, p.key, p.pk0, p.pk1,
                              counter_offset(p) + row * (uint64_t)p.N + (uint64_t)n0, b, h, pp, n0,
                              qw, mw, eo_bits);
  if (L.active) store_block<VEC, LY>(qp, mp, ep, qw, mw, eo_bits);
}

// Update of the model's decode call (ms.py:97-222, 289-544 for the Nemotron-H layout): state rows
// contiguous (row stride N), B and C bf16 with a contiguous d_state, and dt, dt_bias, A and D
// constant within a head (stride 0 along head_dim, A also along d_state), as the model passes
// them. A workgroup of THREADS lanes covers up to R * SLOTS rows of one (batch, head) slice
// (SLOTS = THREADS / (N/16)); lane (slot, blk) owns block column blk of rows slot + r * SLOTS,
// r < R, so B*dt and C are decoded once for R rows and every wave load covers consecutive rows.
// Lane offsets are 32-bit offsets into per-(batch, head) buffer descriptors. Same arithmetic as
// mx_update_kernel in the (B*dt)*x order; in the counter mode rng_offset is a multiple of 16, so a
// block's pair counters are lo0 | k and lowbias32's first step folds into one per-block word.
#ifndef LQ_MX_ROWS_WAVES
#define LQ_MX_ROWS_WAVES 1
#endif

// State blocks and x words of R rows of one lane (the raw loads of one work item).
template <int R>
struct RowLoads {
  uint32_t q[R][4], m[R][2];  // raw block words (layout-dependent, see LayoutOf)
  uint32_t e[R], xw[R], zw[R];
  u32x4_t u[R][4];            // the block's 16 supplied uniforms (LQ_ROUND_SR_UNIFORM only)
};

// Buffer descriptors of one (batch, head) slice.
struct HeadBufs {
  __amdgpu_buffer_rsrc_t q, m, e, x, z, out, u;
};

template <uint32_t N, int LY>
__device__ __forceinline__ HeadBufs head_bufs(const MxUpdateParams& p, int b, int h) {
  using Lay = LayoutOf<LY>;
  HeadBufs hb;
  const uint32_t P = (uint32_t)p.P;
  hb.q = make_buf(p.st.q + (int64_t)b * p.st.qs[0] + (int64_t)h * p.st.qs[1],
                  P * (N / 16) * Lay::qbytes);
  hb.m = make_buf(p.st.mi + (int64_t)b * p.st.ms[0] + (int64_t)h * p.st.ms[1],
                  P * (N / 16) * Lay::mbytes);
  hb.e = make_buf(p.st.e + (int64_t)b * p.st.es[0] + (int64_t)h * p.st.es[1], P * (N / 16));
  hb.x = make_buf(vbase(p.x, b, h), p.x_span);
  hb.z = make_buf(vbase(p.z, b, h), p.z_span);  // span 0 without z: its loads return 0
  hb.out = make_buf(vbase(p.out, b, h), p.out_span);
  hb.u = make_buf(vbase(p.uni, b, h), p.uni_span);  // span 0 outside the uniform mode
  return hb;
}

// Issues the loads of rows row0 + r * SLOTS + slot (clamped to P - 1) of one slice.
// (qo = pc * N + n0 is the block's mantissa offset in the reference layout; every other offset is
// a shift of it.)
template <int R, int SLOTS, uint32_t N, int LY, int RMODE>
__device__ __forceinline__ void load_rows(const MxUpdateParams& p, const HeadBufs& hb, int row0,
                                          int slot, uint32_t n0, RowLoads<R>& L) {
  using Lay = LayoutOf<LY>;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t pc = (uint32_t)min(row0 + r * SLOTS + slot, p.P - 1);
    const uint32_t qo = pc * N + n0;
    if constexpr (Lay::qbytes == 16) {
      const u32x4_t q4 = __builtin_amdgcn_raw_buffer_load_b128(hb.q, qo, 0, STATE_LOAD_POLICY);
      L.q[r][0] = q4.x, L.q[r][1] = q4.y, L.q[r][2] = q4.z, L.q[r][3] = q4.w;
    } else {
      const u32x2_t q2 = __builtin_amdgcn_raw_buffer_load_b64(hb.q, qo >> 1, 0, STATE_LOAD_POLICY);
      L.q[r][0] = q2.x, L.q[r][1] = q2.y, L.q[r][2] = 0, L.q[r][3] = 0;
    }
    if constexpr (Lay::mbits) {
      L.m[r][0] = __builtin_amdgcn_raw_buffer_load_b8(hb.m, qo >> 4, 0, STATE_LOAD_POLICY);
      L.m[r][1] = 0;
    } else {
      const u32x2_t m2 = __builtin_amdgcn_raw_buffer_load_b64(hb.m, qo >> 1, 0, STATE_LOAD_POLICY);
      L.m[r][0] = m2.x, L.m[r][1] = m2.y;
    }
    L.e[r] = __builtin_amdgcn_raw_buffer_load_b8(hb.e, qo >> 4, 0, STATE_LOAD_POLICY);
    L.xw[r] = __builtin_amdgcn_raw_buffer_load_b32(hb.x, (pc * p.x_row_bytes) & ~3u, 0, 0);
    L.zw[r] = __builtin_amdgcn_raw_buffer_load_b32(hb.z, (pc * p.z_row_bytes) & ~3u, 0, 0);
    if constexpr (RMODE == LQ_ROUND_SR_UNIFORM) {
      // the uniforms are read once: streaming loads, issued with the state's
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        L.u[r][j] = __builtin_amdgcn_raw_buffer_load_b128(hb.u, pc * p.uni_row_bytes + n0 * 4u + 16u * j,
                                                          0, STATE_LOAD_POLICY);
      }
    }
  }
}

// Update, y, and writeback encode of the R rows held in L. bdp and cvp point to the lane's 16
// values of B * dt and C in LDS, read again for every row instead of once into 32 VGPRs: the
// compact layouts' 4-row form then fits 74 VGPRs (6 waves per SIMD instead of 5; MX4 at batch 64
// 38.7 -> 37.1 us, batch 128 72.0 -> 68.1 us on one box), the reference layout's 2-row form 67
// (7 waves instead of 6; MX4 at batch 64 39.0-39.2 -> 38.3-38.6 us on one box, three alternated
// runs; with the earlier, VALU-heavier encoder it had been slower, 42.5 against 39.6 us).
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int FB, int RMODE, int BPR_LOG2, int R, int SLOTS, int LY>
__device__ __forceinline__ void update_rows(const MxUpdateParams& p, const HeadBufs& hb, int b,
                                            int h, int row0, int slot, int blk,
                                            const RowLoads<R>& L, const float* bdp,
                                            const float* cvp, const HeadScalars& hs,
                                            const CounterBase& cb, uint64_t poff) {
  constexpr uint32_t N = 16u << BPR_LOG2;
  const uint32_t n0 = (uint32_t)blk * 16u;
  const int P = p.P;
  float Bd[16], Cv[16];
  auto read_bc = [&] {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4_t bq = *(const f32x4_t*)&bdp[4 * i];
      const f32x4_t cq = *(const f32x4_t*)&cvp[4 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Bd[4 * i + j] = bq[j];
        Cv[4 * i + j] = cq[j];
      }
    }
  };
  // x and z of every row converted before the first store: converted inside the row loop, a
  // later row's conversion (a dtype branch) came after the earlier rows' stores, and the wait the
  // compiler placed for its load there (vmcnt counts stores too) also waited for those stores
  float xs[R], zs[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t pc = (uint32_t)min(row0 + r * SLOTS + slot, P - 1);
    xs[r] = word_elem(L.xw[r], ((pc * p.x_row_bytes) & 2u) * 8u, p.x.dtype);
    zs[r] = p.has_z ? word_elem(L.zw[r], ((pc * p.z_row_bytes) & 2u) * 8u, p.z.dtype) : 1.0f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    asm volatile("" ::: "memory");  // keeps the compiler from reusing the previous row's copy
    read_bc();
    const int pp = row0 + r * SLOTS + slot;
    const bool act = pp < P;
    const uint32_t pc = (uint32_t)min(pp, P - 1);
    const float xv = xs[r];
    // h' = h * exp(A dt) + (B dt) x, with the decay folded into the two pair scales (exact)
    const float s0 = pin(__uint_as_float(L.e[r] << 23) * hs.dA);
    const float s1 = pin(__uint_as_float((L.e[r] + 1u) << 23) * hs.dA);
    float hv[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float sk = micro<LY>(L.m[r], k) ? s1 : s0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int n = 2 * k + i;
        hv[n] = fmaf(mant<LY>(L.q[r], n), sk, Bd[n] * xv);
      }
    }
    float ypart = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ypart = fmaf(hv[i], Cv[i], ypart);
    float y = row_sum<BPR_LOG2>(ypart);
    if (p.has_D) y += xv * hs.D;
    y *= zs[r];  // 1.0 without z
    if (act && blk == 0) {
      const uint32_t oo = (uint32_t)pp * p.out_row_bytes;
      if (p.out.dtype == LQ_F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), hb.out, oo, 0, 0);
      } else if (p.out.dtype == LQ_BF16) {  // the hardware's round-to-nearest-even convert
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (__bf16)y), hb.out, oo,
                                              0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)y), hb.out,
                                              oo, 0, 0);
      }
    }

    // writeback encode (ms.py:168-222, 512-544)
    uint32_t qo[4], mo[2], eo;
    if constexpr (RMODE == LQ_ROUND_SR_COUNTER) {
      const uint32_t idx = ((uint32_t)((b * p.H + h) * P + pp) * N + n0) >> 1;
      const uint32_t lo = cb.lo_base + idx;  // the block's first pair counter, low word
      uint32_t base = lo ^ (lo < cb.lo_base ? cb.kh1 : cb.kh);  // its high word carried past hi
      base ^= base >> 16;
      encode16_dither<FB, LY>(hv, HashWords{base}, qo, mo, eo);
    } else if constexpr (RMODE == LQ_ROUND_SR_PHILOX) {
      float u16[16];
      const uint64_t row = ((uint64_t)b * (uint32_t)p.H + (uint32_t)h) * (uint32_t)P + pc;
      philox_block_u16(p.pk0, p.pk1, poff + row * N + n0, u16);
      encode16<FB, LQ_ROUND_SR_UNIFORM, LY>(hv, u16, qo, mo, eo);
    } else {
      float u16[16];
      if constexpr (RMODE == LQ_ROUND_SR_UNIFORM) {
#pragma unroll
        for (int i = 0; i < 16; ++i) u16[i] = __uint_as_float(L.u[r][i >> 2][i & 3]) * 65536.0f;
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) u16[i] = 0.0f;
      }
      encode16<FB, RMODE, LY>(hv, u16, qo, mo, eo);
    }
    if (act) {
      using Lay = LayoutOf<LY>;
      const uint32_t so = (uint32_t)pp * N + n0;
      if constexpr (Lay::qbytes == 16) {
        __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{qo[0], qo[1], qo[2], qo[3]}, hb.q, so, 0,
                                               STATE_STORE_POLICY);
      } else {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{qo[0], qo[1]}, hb.q, so >> 1, 0,
                                              STATE_STORE_POLICY);
      }
      if constexpr (Lay::mbits) {
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)mo[0], hb.m, so >> 4, 0, STATE_STORE_POLICY);
      } else {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{mo[0], mo[1]}, hb.m, so >> 1, 0,
                                              STATE_STORE_POLICY);
      }
      __builtin_amdgcn_raw_buffer_store_b8((uint8_t)eo, hb.e, so >> 4, 0, STATE_STORE_POLICY);
    }
  }
}

// One work item per workgroup: grid (ceil(P / (R * SLOTS)), H, B). Every state load of the lane
// (R state blocks, x, z) is issued before the first use of any of them; B, C and the head scalars
// come through LDS (one barrier).
// The byte-mantissa compact layout (CM8) asks for 6 waves per SIMD: its 4-row form then fits 77-79
// VGPRs without spills instead of taking 84 (5 waves); MX8 at batch 64, three alternated rounds on
// one box: 35.71-35.91 against 36.60-37.33 us. Its supplied-uniform form (2 rows, 256 threads)
// would spill under the cap and keeps the default, as do the other layouts (the nibble layout's
// MX4 form spills at 6 waves).
constexpr int rows_waves(int LY, int RMODE) {
  return LY == LAYOUT_CM8 && RMODE != LQ_ROUND_SR_UNIFORM ? 6 : LQ_MX_ROWS_WAVES;
}
template <int FB, int RMODE, int BPR_LOG2, int R, int THREADS, int LY>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(rows_waves(LY, RMODE))))
void mx_update_rows_kernel(MxUpdateParams p) {
  constexpr int BPR = 1 << BPR_LOG2;
  constexpr uint32_t N = 16 * BPR;
  constexpr int SLOTS = THREADS >> BPR_LOG2;
  const int h = blockIdx.y, b = blockIdx.z;
  const int blk = threadIdx.x & (BPR - 1);
  const int slot = threadIdx.x >> BPR_LOG2;
  const uint32_t n0 = (uint32_t)blk * 16u;
  const int row0 = blockIdx.x * (R * SLOTS);

  const HeadBufs hb = head_bufs<N, LY>(p, b, h);
  constexpr int CONV = (int)N / 2;  // converting threads (see below)
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  // The converting threads' B and C words are loaded before the state: every wave waits at the
  // barrier for them, and issued after the state loads and the head scalars they came back one
  // memory round trip after the state.
  uint32_t bw = 0, cw = 0;
  if (wave * 64 < CONV && (int)threadIdx.x < CONV) {
    const int grp = h / p.ratio;
    const auto rB = make_buf(vbase(p.B, b, grp), N * 2);
    const auto rC = make_buf(vbase(p.C, b, grp), N * 2);
    bw = __builtin_amdgcn_raw_buffer_load_b32(rB, 4u * threadIdx.x, 0, 0);
    cw = __builtin_amdgcn_raw_buffer_load_b32(rC, 4u * threadIdx.x, 0, 0);
  }
  RowLoads<R> L;
  load_rows<R, SLOTS, N, LY, RMODE>(p, hb, row0, slot, n0, L);
  // B * dt and C of the slice as fp32 and the head scalars, computed once per workgroup by the
  // waves that hold the first N / 2 threads (one bf16 pair of B and of C per thread) and shared
  // through LDS: every lane needs 16 of each, and converting them per lane cost about 50 VALU
  // instructions per wave, the head scalars (softplus, exp) about 30 more. The same products as
  // before (B * dt rounded once), so the results are unchanged; at batch 64, MX4, one box: 40.9-41.1
  // -> 40.0-40.3 us, the arithmetic alone (timing-only copy) 36.8 -> 34.6 us.
  __shared__ float s_bd[N], s_c[N], s_hs[2];
  if (wave * 64 < CONV) {  // wave-uniform
    const HeadScalars hs = head_scalars(p, b, h);
    if ((int)threadIdx.x < CONV) {
      const uint32_t t = threadIdx.x;
      s_bd[2 * t] = __uint_as_float(bw << 16) * hs.dt;
      s_bd[2 * t + 1] = __uint_as_float(bw & 0xffff0000u) * hs.dt;
      s_c[2 * t] = __uint_as_float(cw << 16);
      s_c[2 * t + 1] = __uint_as_float(cw & 0xffff0000u);
      if (t == 0) {
        s_hs[0] = hs.dA;
        s_hs[1] = hs.D;
      }
    }
  }
  __syncthreads();
  HeadScalars hs;
  hs.dt = 0.0f;  // folded into B * dt
  hs.dA = s_hs[0];
  hs.D = s_hs[1];
  CounterBase cb{};
  if constexpr (RMODE == LQ_ROUND_SR_COUNTER) cb = counter_base(p);
  uint64_t poff = 0;
  if constexpr (RMODE == LQ_ROUND_SR_PHILOX) poff = counter_offset(p);
  update_rows<FB, RMODE, BPR_LOG2, R, SLOTS, LY>(p, hb, b, h, row0, slot, blk, L, &s_bd[n0],
                                                 &s_c[n0], hs, cb, poff);
}

template <int FB, int RMODE, bool VEC, int LY>
__global__ __launch_bounds__(256) void mx_encode_kernel(MxCodecParams p) {
  const LaneIdx L = lane_index(p.P, p.vbpr_log2, p.bpr);
  if (!L.active) return;
  const int b = L.b, h = L.h, pp = L.pp;
  const int n0 = L.blk * 16;
  float v[16];
  const char* vb = vbase(p.v, b, h);
  const int voff = pp * (int)p.v.s[2] + n0 * (int)p.v.s[3];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = ldf(vb, p.v.dtype, voff + i * (int)p.v.s[3]);
  const uint64_t row = ((uint64_t)b * p.H + h) * p.P + pp;
  uint32_t qw[4], mw[2], eb;
  encode_block<FB, RMODE, LY>(v, p.uni, p.key, p.pk0, p.pk1,
                              p.rng_offset + row * (uint64_t)p.N + (uint64_t)n0, b, h, pp, n0, qw,
                              mw, eb);
  int8_t* qp;
  uint8_t *mp, *ep;
  block_ptrs<LY>(p.st, b, h, pp, L.blk, qp, mp, ep);
  store_block<VEC, LY>(qp, mp, ep, qw, mw, eb);
}

template <bool VEC, int LY>
__global__ __launch_bounds__(256) void mx_decode_kernel(MxCodecParams p) {
  const LaneIdx L = lane_index(p.P, p.vbpr_log2, p.bpr);
  if (!L.active) return;
  const int b = L.b, h = L.h, pp = L.pp;
  const int n0 = L.blk * 16;
  int8_t* qp;
  uint8_t *mp, *ep;
  block_ptrs<LY>(p.st, b, h, pp, L.blk, qp, mp, ep);
  uint32_t qw[4], mw[2], ev;
  load_block<VEC, LY>(qp, mp, ep, qw, mw, ev);
  float hv[16];
  decode16<LY>(qw, mw, ev, hv);
  char* ob = (char*)vbase(p.v, b, h);
  const int off = pp * (int)p.v.s[2] + n0 * (int)p.v.s[3];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int idx = off + i * (int)p.v.s[3];
    if (p.v.dtype == LQ_BF16) {
      ((uint16_t*)ob)[idx] = float_to_bf16_bits(hv[i]);
    } else {
      ((float*)ob)[idx] = hv[i];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------------------------
static uint32_t lowbias32_host(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Per-seed key of the counter generator: K = lowbias32(seed_lo ^ lowbias32(seed_hi ^ 0x9E3779B9)).
static uint32_t seed_key(uint64_t seed) {
  return lowbias32_host((uint32_t)seed ^ lowbias32_host((uint32_t)(seed >> 32) ^ 0x9E3779B9u));
}

// Validates the three MX state tensors and finds their layout from the shapes: with
// NB = shared_exp.shape[3] blocks per row (N = 16 NB values), q_state is [B,H,P,N] (one byte per
// mantissa) or [B,H,P,N/2] (MX4 nibbles), micro_exp [B,H,P,N/2] (one byte per pair) or
// [B,H,P,NB] (bits): reference = bytes + bytes, compact MX8 = bytes + bits, compact MX4 =
// nibbles + bits. `vec`: q and micro blocks aligned for vector access.
static int check_state(const lq_tensor* q, const lq_tensor* e, const lq_tensor* m, int64_t& Bn,
                       int64_t& H, int64_t& P, int64_t& N, MxState& st, bool& vec, int& layout) {
  int rc;
  if ((rc = check_tensor(q, "q_state", 4, false)) != LQ_OK) return rc;
  if ((rc = check_tensor(e, "shared_exp", 4, false, LQ_U8)) != LQ_OK) return rc;
  if ((rc = check_tensor(m, "micro_exp", 4, false, LQ_U8)) != LQ_OK) return rc;
  Bn = e->shape[0];
  H = e->shape[1];
  P = e->shape[2];
  N = 16 * e->shape[3];
  if (N / 16 > 64) {
    return fail(LQ_ERR_UNSUPPORTED, "MX state dim %lld exceeds 1024", (long long)N);
  }
  const int64_t qn = q->shape[3];
  const bool qnib = qn * 2 == N && N > 0;
  if (qn != N && !qnib) {
    if (qn % 16 != 0) {
      return fail(LQ_ERR_INVALID_ARG, "MX state dim must be divisible by 16, got %lld", (long long)qn);
    }
    return fail(LQ_ERR_INVALID_ARG,
                "q_state must be [B, H, P, N] or, MX4 nibbles, [B, H, P, N/2] (N = 16 * shared_exp dim)");
  }
  const bool mbits = m->shape[3] == N / 16;
  if (!mbits && m->shape[3] != N / 2) {
    return fail(LQ_ERR_INVALID_ARG, "micro_exp must be [B, H, P, N/2] or, bits, [B, H, P, N/16]");
  }
  if (qnib && !mbits) {
    return fail(LQ_ERR_INVALID_ARG, "nibble mantissas need bit micro-exponents [B, H, P, N/16]");
  }
  layout = qnib ? LAYOUT_CM4 : (mbits ? LAYOUT_CM8 : LAYOUT_REF);
  if (layout == LAYOUT_REF && q->dtype != LQ_I8) {
    return fail(LQ_ERR_INVALID_ARG, "q_state: dtype code %d, expected %d", q->dtype, LQ_I8);
  }
  if (q->dtype != LQ_I8 && q->dtype != LQ_U8) {
    return fail(LQ_ERR_INVALID_ARG, "q_state: dtype code %d, expected int8 or uint8", q->dtype);
  }
  for (int i = 0; i < 3; ++i) {
    if (q->shape[i] != e->shape[i] || m->shape[i] != e->shape[i]) {
      return fail(LQ_ERR_INVALID_ARG, "q_state, shared_exp and micro_exp must share [B, H, P]");
    }
  }
  if (q->stride[3] != 1 || e->stride[3] != 1 || m->stride[3] != 1) {
    return fail(LQ_ERR_INVALID_ARG, "MX state tensors need a contiguous last dimension");
  }
  st.q = (int8_t*)q->data;
  st.e = (uint8_t*)e->data;
  st.mi = (uint8_t*)m->data;
  const int qa = qnib ? 8 : 16;
  const int ma = mbits ? 1 : 8;
  vec = (((uintptr_t)st.q % qa) == 0) && (((uintptr_t)st.mi % ma) == 0);
  for (int i = 0; i < 3; ++i) {
    st.qs[i] = q->stride[i];
    st.es[i] = e->stride[i];
    st.ms[i] = m->stride[i];
    vec = vec && (st.qs[i] % qa == 0) && (st.ms[i] % ma == 0);
  }
  return LQ_OK;
}

static int check_round(int format_bits, int round_mode, const lq_tensor* uniform, int64_t Bn,
                       int64_t H, int64_t P, int64_t N, uint64_t rng_offset) {
  if (format_bits != 8 && format_bits != 4) {
    return fail(LQ_ERR_INVALID_ARG, "Unsupported MX state format_bits=%d", format_bits);
  }
  if (round_mode < LQ_ROUND_NEAREST_EVEN || round_mode > LQ_ROUND_SR_PHILOX) {
    return fail(LQ_ERR_INVALID_ARG, "unknown round_mode %d", round_mode);
  }
  if (round_mode == LQ_ROUND_SR_UNIFORM) {
    int rc;
    if ((rc = check_tensor(uniform, "uniform", 4, false, LQ_F32)) != LQ_OK) return rc;
    const int64_t want[4] = {Bn, H, P, N};
    for (int i = 0; i < 4; ++i) {
      if (uniform->shape[i] != want[i]) {
        return fail(LQ_ERR_INVALID_ARG, "uniform must be [B, H, P, N]");
      }
    }
  }
  if (round_mode == LQ_ROUND_SR_COUNTER && (rng_offset & 1u) != 0) {
    return fail(LQ_ERR_INVALID_ARG, "rng_offset must be even");
  }
  return LQ_OK;
}

static int check_shape3(const lq_tensor* t, const char* name, int64_t a, int64_t b, int64_t c,
                        bool allow_null) {
  if (t == nullptr && allow_null) return LQ_OK;
  int rc;
  if ((rc = check_tensor(t, name, 3, true)) != LQ_OK) return rc;
  if (t->shape[0] != a || t->shape[1] != b || t->shape[2] != c) {
    return fail(LQ_ERR_INVALID_ARG, "Expected %s shape (%lld, %lld, %lld), got (%lld, %lld, %lld)",
                name, (long long)a, (long long)b, (long long)c, (long long)t->shape[0],
                (long long)t->shape[1], (long long)t->shape[2]);
  }
  return LQ_OK;
}

static int check_shape2(const lq_tensor* t, const char* name, int64_t a, int64_t b) {
  if (t == nullptr) return LQ_OK;
  int rc;
  if ((rc = check_tensor(t, name, 2, true)) != LQ_OK) return rc;
  if (t->shape[0] != a || t->shape[1] != b) {
    return fail(LQ_ERR_INVALID_ARG, "Expected %s shape (%lld, %lld)", name, (long long)a,
                (long long)b);
  }
  return LQ_OK;
}

// Lane offsets below the (batch, head) level are 32-bit: the span of dims >= first must fit.
static bool lane_span_ok(const lq_tensor* t, int first) {
  if (t == nullptr) return true;
  int64_t span = 0;
  for (int i = 0; i < t->ndim; ++i) {
    if (t->stride[i] < 0) return false;
    if (i >= first && t->shape[i] > 0) span += (t->shape[i] - 1) * t->stride[i];
  }
  return span < ((int64_t)1 << 31) - 64;
}

static int log2_ceil(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

static bool bc_vector_ok(const lq_tensor* t) {
  return t->dtype == LQ_BF16 && t->stride[2] == 1 && ((uintptr_t)t->data & 15) == 0 &&
         t->stride[0] % 8 == 0 && t->stride[1] % 8 == 0;
}

// Calls f(std::integral_constant<int, LY>) for the layout code (compact MX4 only with 4-bit
// mantissas, which the nibbles can hold); returns an error for an impossible combination.
template <int FB, class F>
static int with_layout(int layout, F&& f) {
  switch (layout) {
    case LAYOUT_REF: f(std::integral_constant<int, LAYOUT_REF>{}); return LQ_OK;
    case LAYOUT_CM8: f(std::integral_constant<int, LAYOUT_CM8>{}); return LQ_OK;
    default:
      if constexpr (FB == 4) {
        f(std::integral_constant<int, LAYOUT_CM4>{});
        return LQ_OK;
      } else {
        return fail(LQ_ERR_INVALID_ARG,
                    "nibble mantissas hold MX4 only (format_bits=8 needs [B, H, P, N] q_state)");
      }
  }
}

template <int FB, int RMODE, int LY>
static void launch_update(const MxUpdateParams& p, bool vec, bool bcvec, dim3 grid,
                          hipStream_t st) {
  if (vec && bcvec) {
    hipLaunchKernelGGL((mx_update_kernel<FB, RMODE, true, true, LY>), grid, dim3(256), 0, st, p);
  } else if (vec) {
    hipLaunchKernelGGL((mx_update_kernel<FB, RMODE, true, false, LY>), grid, dim3(256), 0, st, p);
  } else if (bcvec) {
    hipLaunchKernelGGL((mx_update_kernel<FB, RMODE, false, true, LY>), grid, dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((mx_update_kernel<FB, RMODE, false, false, LY>), grid, dim3(256), 0, st, p);
  }
}

template <int FB, int LY>
static void dispatch_update(const MxUpdateParams& p, int rmode, bool vec, bool bcvec, dim3 grid,
                            hipStream_t st) {
  switch (rmode) {
    case LQ_ROUND_NEAREST_EVEN:
      launch_update<FB, LQ_ROUND_NEAREST_EVEN, LY>(p, vec, bcvec, grid, st);
      break;
    case LQ_ROUND_HALF_UP: launch_update<FB, LQ_ROUND_HALF_UP, LY>(p, vec, bcvec, grid, st); break;
    case LQ_ROUND_SR_UNIFORM:
      launch_update<FB, LQ_ROUND_SR_UNIFORM, LY>(p, vec, bcvec, grid, st);
      break;
    case LQ_ROUND_SR_PHILOX:
      launch_update<FB, LQ_ROUND_SR_PHILOX, LY>(p, vec, bcvec, grid, st);
      break;
    default: launch_update<FB, LQ_ROUND_SR_COUNTER, LY>(p, vec, bcvec, grid, st); break;
  }
}

template <int FB, int RMODE, int LY>
static void launch_encode(const MxCodecParams& p, bool vec, dim3 grid, hipStream_t st) {
  if (vec) {
    hipLaunchKernelGGL((mx_encode_kernel<FB, RMODE, true, LY>), grid, dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((mx_encode_kernel<FB, RMODE, false, LY>), grid, dim3(256), 0, st, p);
  }
}

template <int FB, int LY>
static void dispatch_encode(const MxCodecParams& p, int rmode, bool vec, dim3 grid,
                            hipStream_t st) {
  switch (rmode) {
    case LQ_ROUND_NEAREST_EVEN: launch_encode<FB, LQ_ROUND_NEAREST_EVEN, LY>(p, vec, grid, st); break;
    case LQ_ROUND_HALF_UP: launch_encode<FB, LQ_ROUND_HALF_UP, LY>(p, vec, grid, st); break;
    case LQ_ROUND_SR_UNIFORM: launch_encode<FB, LQ_ROUND_SR_UNIFORM, LY>(p, vec, grid, st); break;
    case LQ_ROUND_SR_PHILOX: launch_encode<FB, LQ_ROUND_SR_PHILOX, LY>(p, vec, grid, st); break;
    default: launch_encode<FB, LQ_ROUND_SR_COUNTER, LY>(p, vec, grid, st); break;
  }
}

// Rows kernel geometry: R rows per lane, THREADS threads, one (batch, head) slice of up to
// R * THREADS / (N/16) rows per workgroup (64 rows = one Nemotron-H head at N = 128). The reference
// layout keeps 2 rows per lane (67 VGPRs, 7 waves per SIMD: its 212 MB per call at batch 64 need
// the waves to hide memory latency; 4 rows per lane take 87 VGPRs, 5 waves, and with an earlier
// build ran 42.2 against 41.4 us). The compact layouts move 2.5x fewer bytes and are bound by their arithmetic, so 4 rows
// per lane share the per-lane setup (head scalars, B and C) over twice the rows: 41.1 -> 38.9 us
// for MX4 at batch 64 (91 VGPRs, 5 waves per SIMD). The supplied-uniform mode keeps 2 rows per
// lane everywhere: its 16 uniforms per row would take 155-161 VGPRs at 4 rows. So does the Philox
// mode, whose 4-row form kept the rows' arrays in scratch memory.
template <int LY, int RMODE>
struct RowsGeometry {
  static constexpr bool wide =
      LY != LAYOUT_REF && RMODE != LQ_ROUND_SR_UNIFORM && RMODE != LQ_ROUND_SR_PHILOX;
  static constexpr int R = wide ? 4 : 2;
  static constexpr int THREADS = wide ? 128 : 256;
  static_assert(R * THREADS == 512, "rows_per_workgroup assumes R * THREADS = 512");
};
// Rows per workgroup: the same for every layout and mode (R * THREADS = 512 lanes' rows).
constexpr int rows_per_workgroup(int vbpr_log2) { return 512 >> vbpr_log2; }

template <int FB, int RMODE, int BPR_LOG2, int LY>
static void launch_rows_mode(const MxUpdateParams& p, dim3 grid, hipStream_t st) {
  using G = RowsGeometry<LY, RMODE>;
  hipLaunchKernelGGL((mx_update_rows_kernel<FB, RMODE, BPR_LOG2, G::R, G::THREADS, LY>), grid,
                     dim3(G::THREADS), 0, st, p);
}

template <int FB, int BPR_LOG2, int LY>
static void launch_rows(const MxUpdateParams& p, int rmode, dim3 grid, hipStream_t st) {
  switch (rmode) {
    case LQ_ROUND_NEAREST_EVEN: launch_rows_mode<FB, LQ_ROUND_NEAREST_EVEN, BPR_LOG2, LY>(p, grid, st); break;
    case LQ_ROUND_HALF_UP: launch_rows_mode<FB, LQ_ROUND_HALF_UP, BPR_LOG2, LY>(p, grid, st); break;
    case LQ_ROUND_SR_UNIFORM: launch_rows_mode<FB, LQ_ROUND_SR_UNIFORM, BPR_LOG2, LY>(p, grid, st); break;
    case LQ_ROUND_SR_PHILOX: launch_rows_mode<FB, LQ_ROUND_SR_PHILOX, BPR_LOG2, LY>(p, grid, st); break;
    default: launch_rows_mode<FB, LQ_ROUND_SR_COUNTER, BPR_LOG2, LY>(p, grid, st); break;
  }
}

template <int FB, int LY>
static void dispatch_rows(const MxUpdateParams& p, int rmode, dim3 grid, hipStream_t st) {
  switch (p.vbpr_log2) {
    case 2: launch_rows<FB, 2, LY>(p, rmode, grid, st); break;
    case 3: launch_rows<FB, 3, LY>(p, rmode, grid, st); break;
    default: launch_rows<FB, 4, LY>(p, rmode, grid, st); break;
  }
}

// The rows kernel's preconditions (else the general kernel runs): d_state 64, 128 or 256;
// vector-aligned state with contiguous rows; bf16 B/C with contiguous d_state; dt, dt_bias, A, D
// constant within a head; in the counter mode rng_offset a multiple of 16 (then so is every
// offset with a device step, whose stride B*H*P*N is a multiple of 16) and fewer than 2^32 state
// elements.
static bool rows_path_ok(const MxUpdateParams& p, bool vec, bool bcvec, const lq_tensor* dt,
                         const lq_tensor* dt_bias, const lq_tensor* A, const lq_tensor* D,
                         int round_mode, int64_t total, int layout) {
  if (diag(LQ_DIAG_MX_FORCE_GENERIC)) return false;
  if (!vec || !bcvec) return false;
  if (p.N != 64 && p.N != 128 && p.N != 256) return false;
  const int64_t q_row = layout == LAYOUT_CM4 ? p.N / 2 : p.N;
  const int64_t m_row = layout == LAYOUT_REF ? p.N / 2 : p.N / 16;
  if (p.st.qs[2] != q_row || p.st.ms[2] != m_row || p.st.es[2] != p.N / 16) return false;
  if (dt->stride[2] != 0 || A->stride[1] != 0 || A->stride[2] != 0) return false;
  // byte offsets of x, z and out rows within a (batch, head) slice are 32-bit
  const int64_t lim = (int64_t)1 << 28;
  if (p.P * p.x.s[2] >= lim || p.P * p.out.s[2] >= lim || p.P * p.z.s[2] >= lim) return false;
  if (p.x.s[2] < 0 || p.out.s[2] < 0 || p.z.s[2] < 0) return false;
  if (dt_bias != nullptr && dt_bias->stride[1] != 0) return false;
  if (D != nullptr && D->stride[1] != 0) return false;
  if (round_mode == LQ_ROUND_SR_UNIFORM) {
    // contiguous along d_state, 16-byte aligned rows, 32-bit slice spans
    const View& u = p.uni;
    if (u.s[3] != 1 || u.s[2] < p.N || (u.s[2] * 4) % 16 != 0 || u.s[0] % 4 != 0 || u.s[1] % 4 != 0) {
      return false;
    }
    if (((uintptr_t)u.data & 15) != 0) return false;
    if (((p.P - 1) * u.s[2] + p.N) * 4 >= lim) return false;
  }
  if (round_mode == LQ_ROUND_SR_COUNTER) {
    if (p.rng_offset % 16 != 0 || total >= ((int64_t)1 << 32)) return false;
  }
  return true;
}

static int grid_for(int64_t Bn, int64_t H, int64_t P, int vbpr_log2, dim3& grid) {
  if (Bn > 65535 || H > 65535) {
    return fail(LQ_ERR_UNSUPPORTED, "batch %lld or heads %lld exceed 65535", (long long)Bn,
                (long long)H);
  }
  const int64_t lanes = P << vbpr_log2;
  if (lanes >= ((int64_t)1 << 31) - 256) {
    return fail(LQ_ERR_UNSUPPORTED, "head_dim %lld too large", (long long)P);
  }
  grid = dim3((unsigned)((lanes + 255) / 256), (unsigned)H, (unsigned)Bn);
  return LQ_OK;
}

}  // namespace lq

using namespace lq;

static int mx_state_update(const lq_tensor* q_state, const lq_tensor* shared_exp,
                           const lq_tensor* micro_exp, const lq_tensor* x, const lq_tensor* dt,
                           const lq_tensor* dt_bias, const lq_tensor* A, const lq_tensor* B,
                           const lq_tensor* C, const lq_tensor* D, const lq_tensor* z,
                           const lq_tensor* out, int format_bits, int dt_softplus, int round_mode,
                           const lq_tensor* uniform, uint64_t seed, uint64_t rng_offset,
                           const lq_tensor* step, void* stream) {
  int rc;
  int64_t Bn, H, P, N;
  MxState st{};
  bool vec = false;
  int layout = LAYOUT_REF;
  if ((rc = check_state(q_state, shared_exp, micro_exp, Bn, H, P, N, st, vec, layout)) != LQ_OK) {
    return rc;
  }
  if ((rc = check_shape3(x, "x", Bn, H, P, false)) != LQ_OK) return rc;
  if (B == nullptr || C == nullptr || B->ndim != 3 || C->ndim != 3) {
    return fail(LQ_ERR_INVALID_ARG,
                "Expected B and C with shape [batch, ngroups, dstate] for decode update.");
  }
  if ((rc = check_tensor(B, "B", 3, true)) != LQ_OK) return rc;
  if ((rc = check_tensor(C, "C", 3, true)) != LQ_OK) return rc;
  const int64_t G = B->shape[1];
  if (B->shape[0] != Bn || B->shape[2] != N || C->shape[0] != Bn || C->shape[1] != G ||
      C->shape[2] != N) {
    return fail(LQ_ERR_INVALID_ARG,
                "Expected B and C with shape [batch, ngroups, dstate] for decode update.");
  }
  if (G <= 0 || H % G != 0) {
    return fail(LQ_ERR_INVALID_ARG, "nheads=%lld not divisible by ngroups=%lld", (long long)H,
                (long long)G);
  }
  if ((rc = check_shape3(dt, "dt", Bn, H, P, false)) != LQ_OK) return rc;
  if ((rc = check_shape3(z, "z", Bn, H, P, true)) != LQ_OK) return rc;
  if ((rc = check_shape3(out, "out", Bn, H, P, false)) != LQ_OK) return rc;
  if ((rc = check_shape2(dt_bias, "dt_bias", H, P)) != LQ_OK) return rc;
  if ((rc = check_shape2(D, "D", H, P)) != LQ_OK) return rc;
  if ((rc = check_tensor(A, "A", 3, true)) != LQ_OK) return rc;
  if (A->shape[0] != H || A->shape[1] != P || A->shape[2] != N) {
    return fail(LQ_ERR_INVALID_ARG, "Expected A shape (%lld, %lld, %lld)", (long long)H,
                (long long)P, (long long)N);
  }
  if ((rc = check_round(format_bits, round_mode, uniform, Bn, H, P, N, rng_offset)) != LQ_OK) {
    return rc;
  }
  if (step != nullptr) {
    if ((rc = check_tensor(step, "step", 1, false, LQ_I64)) != LQ_OK) return rc;
    if (step->shape[0] < 1) return fail(LQ_ERR_INVALID_ARG, "step must hold one value");
    if (((uintptr_t)step->data & 7) != 0) return fail(LQ_ERR_INVALID_ARG, "step must be 8-byte aligned");
  }
  if (Bn == 0 || H == 0 || P == 0) return LQ_OK;

  MxUpdateParams p{};
  p.st = st;
  p.x = make_view(x);
  p.dt = make_view(dt);
  p.dtb = make_view(dt_bias);
  p.A = make_view(A);
  p.B = make_view(B);
  p.C = make_view(C);
  p.D = make_view(D);
  p.z = make_view(z);
  p.out = make_view(out);
  p.uni = make_view(round_mode == LQ_ROUND_SR_UNIFORM ? uniform : nullptr);
  p.Bn = (int)Bn;
  p.H = (int)H;
  p.P = (int)P;
  p.N = (int)N;
  p.ratio = (int)(H / G);
  p.bpr = (int)(N / 16);
  p.vbpr_log2 = log2_ceil(p.bpr);
  p.has_dtb = dt_bias != nullptr;
  p.has_D = D != nullptr;
  p.has_z = z != nullptr;
  p.softplus = dt_softplus != 0;
  p.a_row_const = A->stride[2] == 0;
  p.key = seed_key(seed);
  p.pk0 = (uint32_t)seed;
  p.pk1 = (uint32_t)(seed >> 32);
  p.rng_offset = rng_offset;
  if (step != nullptr && (round_mode == LQ_ROUND_SR_COUNTER || round_mode == LQ_ROUND_SR_PHILOX)) {
    p.step_dev = (const int64_t*)step->data;
    p.step_stride = (uint64_t)(Bn * H * P * N);
  }

  const lq_tensor* spans[] = {q_state, shared_exp, micro_exp, x, dt, B, C, z, out, uniform};
  for (const lq_tensor* t : spans) {
    if (!lane_span_ok(t, 2)) return fail(LQ_ERR_UNSUPPORTED, "tensor spans exceed 32-bit offsets");
  }
  if (!lane_span_ok(A, 1) || !lane_span_ok(D, 1) || !lane_span_ok(dt_bias, 1)) {
    return fail(LQ_ERR_UNSUPPORTED, "tensor spans exceed 32-bit offsets");
  }
  dim3 grid;
  if ((rc = grid_for(Bn, H, P, p.vbpr_log2, grid)) != LQ_OK) return rc;
  const bool bcvec = bc_vector_ok(B) && bc_vector_ok(C);
  hipStream_t s = (hipStream_t)stream;
  if (layout == LAYOUT_CM4 && format_bits != 4) {
    return fail(LQ_ERR_INVALID_ARG,
                "nibble mantissas hold MX4 only (format_bits=8 needs [B, H, P, N] q_state)");
  }
  if (rows_path_ok(p, vec, bcvec, dt, dt_bias, A, D, round_mode, Bn * H * P * N, layout)) {
    p.lo_base = (uint32_t)(rng_offset >> 1);
    p.kh = lowbias32_host((uint32_t)(rng_offset >> 33) ^ p.key);
    p.kh1 = lowbias32_host(((uint32_t)(rng_offset >> 33) + 1u) ^ p.key);
    // per-row byte strides and slice spans of x, z and out
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
    if (round_mode == LQ_ROUND_SR_UNIFORM) {
      p.uni_row_bytes = (uint32_t)(p.uni.s[2] * 4);
      p.uni_span = (uint32_t)(((P - 1) * p.uni.s[2] + N) * 4);
    } else {  // a zero-span descriptor: never read
      p.uni = p.x;
      p.uni_row_bytes = 0;
      p.uni_span = 0;
    }
    // absent dt_bias or D: read dt's first element instead (the value is not used)
    const View dt0{p.dt.data, p.dt.dtype, {0, 0, 0, 0}};
    if (!p.has_dtb) p.dtb = dt0;
    if (!p.has_D) p.D = dt0;
    const int rows = rows_per_workgroup(p.vbpr_log2);
    const dim3 rgrid((unsigned)((P + rows - 1) / rows), (unsigned)H, (unsigned)Bn);
    if (format_bits == 8) {
      rc = with_layout<8>(layout, [&](auto ly) { dispatch_rows<8, ly()>(p, round_mode, rgrid, s); });
    } else {
      rc = with_layout<4>(layout, [&](auto ly) { dispatch_rows<4, ly()>(p, round_mode, rgrid, s); });
    }
    if (rc != LQ_OK) return rc;
    return check_launch("lq_mx_state_update");
  }
  if (diag(LQ_DIAG_MX_REQUIRE_ROWS)) {  // tests: the call must take the row kernel
    return fail(LQ_ERR_INVALID_ARG,
                "LQ_MX_REQUIRE_ROWS is set and this call's layout takes the general kernel");
  }
  if (format_bits == 8) {
    rc = with_layout<8>(layout,
                        [&](auto ly) { dispatch_update<8, ly()>(p, round_mode, vec, bcvec, grid, s); });
  } else {
    rc = with_layout<4>(layout,
                        [&](auto ly) { dispatch_update<4, ly()>(p, round_mode, vec, bcvec, grid, s); });
  }
  if (rc != LQ_OK) return rc;
  return check_launch("lq_mx_state_update");
}

extern "C" int lq_mx_state_update(const lq_tensor* q_state, const lq_tensor* shared_exp,
                                  const lq_tensor* micro_exp, const lq_tensor* x,
                                  const lq_tensor* dt, const lq_tensor* dt_bias,
                                  const lq_tensor* A, const lq_tensor* B, const lq_tensor* C,
                                  const lq_tensor* D, const lq_tensor* z, const lq_tensor* out,
                                  int format_bits, int dt_softplus, int round_mode,
                                  const lq_tensor* uniform, uint64_t seed, uint64_t rng_offset,
                                  void* stream) {
  return mx_state_update(q_state, shared_exp, micro_exp, x, dt, dt_bias, A, B, C, D, z, out,
                         format_bits, dt_softplus, round_mode, uniform, seed, rng_offset, nullptr,
                         stream);
}

extern "C" int lq_mx_state_update_device_step(
    const lq_tensor* q_state, const lq_tensor* shared_exp, const lq_tensor* micro_exp,
    const lq_tensor* x, const lq_tensor* dt, const lq_tensor* dt_bias, const lq_tensor* A,
    const lq_tensor* B, const lq_tensor* C, const lq_tensor* D, const lq_tensor* z,
    const lq_tensor* out, int format_bits, int dt_softplus, int round_mode,
    const lq_tensor* uniform, uint64_t seed, uint64_t rng_offset, const lq_tensor* step,
    void* stream) {
  if (step == nullptr) return fail(LQ_ERR_INVALID_ARG, "step: descriptor is NULL");
  return mx_state_update(q_state, shared_exp, micro_exp, x, dt, dt_bias, A, B, C, D, z, out,
                         format_bits, dt_softplus, round_mode, uniform, seed, rng_offset, step,
                         stream);
}

extern "C" int lq_mx_encode(const lq_tensor* state, const lq_tensor* q_state,
                            const lq_tensor* shared_exp, const lq_tensor* micro_exp,
                            int format_bits, int round_mode, const lq_tensor* uniform,
                            uint64_t seed, uint64_t rng_offset, void* stream) {
  int rc;
  int64_t Bn, H, P, N;
  MxState st{};
  bool vec = false;
  int layout = LAYOUT_REF;
  if ((rc = check_state(q_state, shared_exp, micro_exp, Bn, H, P, N, st, vec, layout)) != LQ_OK) {
    return rc;
  }
  if ((rc = check_tensor(state, "state", 4, true)) != LQ_OK) return rc;
  for (int i = 0; i < 4; ++i) {
    const int64_t want[4] = {Bn, H, P, N};
    if (state->shape[i] != want[i]) {
      return fail(LQ_ERR_INVALID_ARG, "state must match q_state [B, H, P, N]");
    }
  }
  if ((rc = check_round(format_bits, round_mode, uniform, Bn, H, P, N, rng_offset)) != LQ_OK) {
    return rc;
  }
  if (Bn == 0 || H == 0 || P == 0) return LQ_OK;
  MxCodecParams p{};
  p.st = st;
  p.v = make_view(state);
  p.uni = make_view(round_mode == LQ_ROUND_SR_UNIFORM ? uniform : nullptr);
  p.Bn = (int)Bn;
  p.H = (int)H;
  p.P = (int)P;
  p.N = (int)N;
  p.bpr = (int)(N / 16);
  p.vbpr_log2 = log2_ceil(p.bpr);
  p.key = seed_key(seed);
  p.pk0 = (uint32_t)seed;
  p.pk1 = (uint32_t)(seed >> 32);
  p.rng_offset = rng_offset;
  const lq_tensor* spans[] = {q_state, shared_exp, micro_exp, state, uniform};
  for (const lq_tensor* t : spans) {
    if (!lane_span_ok(t, 2)) return fail(LQ_ERR_UNSUPPORTED, "tensor spans exceed 32-bit offsets");
  }
  dim3 grid;
  if ((rc = grid_for(Bn, H, P, p.vbpr_log2, grid)) != LQ_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (layout == LAYOUT_CM4 && format_bits != 4) {
    return fail(LQ_ERR_INVALID_ARG,
                "nibble mantissas hold MX4 only (format_bits=8 needs [B, H, P, N] q_state)");
  }
  if (format_bits == 8) {
    rc = with_layout<8>(layout, [&](auto ly) { dispatch_encode<8, ly()>(p, round_mode, vec, grid, s); });
  } else {
    rc = with_layout<4>(layout, [&](auto ly) { dispatch_encode<4, ly()>(p, round_mode, vec, grid, s); });
  }
  if (rc != LQ_OK) return rc;
  return check_launch("lq_mx_encode");
}

extern "C" int lq_mx_decode(const lq_tensor* q_state, const lq_tensor* shared_exp,
                            const lq_tensor* micro_exp, const lq_tensor* out, void* stream) {
  int rc;
  int64_t Bn, H, P, N;
  MxState st{};
  bool vec = false;
  int layout = LAYOUT_REF;
  if ((rc = check_state(q_state, shared_exp, micro_exp, Bn, H, P, N, st, vec, layout)) != LQ_OK) {
    return rc;
  }
  if ((rc = check_tensor(out, "out", 4, true)) != LQ_OK) return rc;
  for (int i = 0; i < 4; ++i) {
    const int64_t want[4] = {Bn, H, P, N};
    if (out->shape[i] != want[i]) {
      return fail(LQ_ERR_INVALID_ARG, "out must match q_state [B, H, P, N]");
    }
  }
  if (Bn == 0 || H == 0 || P == 0) return LQ_OK;
  MxCodecParams p{};
  p.st = st;
  p.v = make_view(out);
  p.Bn = (int)Bn;
  p.H = (int)H;
  p.P = (int)P;
  p.N = (int)N;
  p.bpr = (int)(N / 16);
  p.vbpr_log2 = log2_ceil(p.bpr);
  const lq_tensor* spans[] = {q_state, shared_exp, micro_exp, out};
  for (const lq_tensor* t : spans) {
    if (!lane_span_ok(t, 2)) return fail(LQ_ERR_UNSUPPORTED, "tensor spans exceed 32-bit offsets");
  }
  dim3 grid;
  if ((rc = grid_for(Bn, H, P, p.vbpr_log2, grid)) != LQ_OK) return rc;
  rc = with_layout<4>(layout, [&](auto ly) {
    if (vec) {
      hipLaunchKernelGGL((mx_decode_kernel<true, ly()>), grid, dim3(256), 0, (hipStream_t)stream, p);
    } else {
      hipLaunchKernelGGL((mx_decode_kernel<false, ly()>), grid, dim3(256), 0, (hipStream_t)stream, p);
    }
  });
  if (rc != LQ_OK) return rc;
  return check_launch("lq_mx_decode");
}
