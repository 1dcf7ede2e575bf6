/*
 * layer_quant.h -- C ABI of the MI355X (gfx950) decode-path kernels.
 *
 * One shared library (liblayer_quant.so) exports the entry points below. They replace the
 * Triton kernel launches of the reference's two quantized decode paths:
 *
 *   hybrid_quant/int4_8b_attention.py     INT4 KV cache: per-token pack, q_len=1 decode attention
 *                                         and causal prefill attention over the packed cache
 *   hybrid_quant/mamba_state_8b_kernel.py Mamba2 selective-state update over an MX8/MX4 state
 *
 * Conventions
 *   - The caller owns every buffer. The library never allocates device memory; scratch space
 *     (split-K partials) comes from a caller workspace sized by a query function, or, for
 *     lq_int4_decode_attention_noalloc, from a static 8 MiB buffer per device that the library's
 *     code object holds from load to process end.
 *   - Every launch is asynchronous on the caller's HIP stream, passed as `void* stream`
 *     (a hipStream_t; NULL is the legacy default stream). No entry point synchronizes.
 *   - Tensors are described by lq_tensor: a device pointer, a dtype code, a rank (1..4), a shape
 *     and strides counted in ELEMENTS (not bytes). Strides may be 0 (broadcast views).
 *   - Return value: 0 on success, a negative LQ_ERR_* code on failure. lq_last_error() returns a
 *     thread-local message describing the last failure on the calling thread. Argument
 *     validation happens before any HIP call, so invalid arguments never touch the device.
 */
#ifndef LAYER_QUANT_H_
#define LAYER_QUANT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LQ_ABI_VERSION 1

/* dtype codes for lq_tensor.dtype */
enum {
  LQ_U8 = 0,
  LQ_I8 = 1,
  LQ_F16 = 2,
  LQ_BF16 = 3,
  LQ_F32 = 4,
  LQ_I32 = 5,
  LQ_I64 = 6
};

/* error codes */
enum {
  LQ_OK = 0,
  LQ_ERR_INVALID_ARG = -1,
  LQ_ERR_UNSUPPORTED = -2,
  LQ_ERR_WORKSPACE = -3,
  LQ_ERR_HIP = -4
};

/* rounding modes of the MX encoders */
enum {
  LQ_ROUND_NEAREST_EVEN = 0, /* torch.round of clamp(|v|/scale, 0, M): the initial encode       */
  LQ_ROUND_HALF_UP = 1,      /* floor(min(|v|/scale, M) + 0.5): the deterministic writeback     */
  LQ_ROUND_SR_UNIFORM = 2,   /* floor(q) + (u < q - floor(q)), u from a caller fp32 tensor       */
  LQ_ROUND_SR_COUNTER = 3,   /* stochastic, 16-bit draws of the library's counter generator:    */
                             /* floor(RN_{2^-16}(v/scale + u)), u = u16 * 2^-16 (see below)     */
  LQ_ROUND_SR_PHILOX = 4     /* floor(q) + (u < q - floor(q)), u = the reference's own draw     */
                             /* tl.rand(seed, offset): Triton's Philox4x32-10 (see below)      */
};
/*
 * The counter-based generator of LQ_ROUND_SR_COUNTER: element (b,h,p,n) draws counter
 * c = rng_offset + ((b*H + h)*P + p)*N + n (the reference's tl.rand offsets, step*B*H*P*N + index,
 * when rng_offset = step*B*H*P*N). With K = lowbias32(lo32(seed) ^ lowbias32(hi32(seed) ^
 * 0x9E3779B9)) and W = lowbias32(lo32(c>>1) ^ lowbias32(hi32(c>>1) ^ K)), the draw is
 * u16 = (W >> 16*(c&1)) & 0xFFFF. With qs = v / pair_scale (exact) the level is
 * floor(t) - 192, t = fp32(192 + u16 * 2^-16 + qs) clamped to [192 - M, 193 + M - 2^-16]: qs plus
 * the draw rounded to the 2^-16 grid (ties to even), floored, so |v| rounds up with probability
 * round(frac(|qs|) * 2^16) / 2^16 (bias within 2^-17 of a level step).
 * lowbias32(x): x ^= x>>16; x *= 0x7feb352d; x ^= x>>15; x *= 0x846ca68b; x ^= x>>16.
 *
 * LQ_ROUND_SR_PHILOX reproduces the reference's stochastic writeback, u = tl.rand(RNG_SEED,
 * RNG_OFFSET + index) (hybrid_quant/mamba_state_8b_kernel.py:198, 405, 479, 529; Triton's
 * triton/language/random.py), bit for bit: element (b,h,p,n) takes offset
 * c = rng_offset + ((b*H + h)*P + p)*N + n and runs Philox4x32 with 10 rounds on the counter
 * (lo32(c), hi32(c), 0, 0) under the key (lo32(seed), hi32(seed)):
 *   c0' = mulhi(0xCD9E8D57, c2) ^ c1 ^ k0;  c1' = 0xCD9E8D57 * c2;
 *   c2' = mulhi(0xD2511F53, c0) ^ c3 ^ k1;  c3' = 0xD2511F53 * c0;  k0 += 0x9E3779B9;
 *   k1 += 0xBB67AE85.  With x = (int32) c0 after the last round, u = fp32(x < 0 ? -x-1 : x) *
 *   0x1.fffffep-32 in [0, 1 - 2^-24]. The level is floor(q) + (u < q - floor(q)), as in
 *   LQ_ROUND_SR_UNIFORM. (The reference's offsets are int32: they agree with c wherever its
 *   kernels compile.) About 2.7x the counter mode's time: a fidelity mode.
 */

typedef struct lq_tensor {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[4];
  int64_t stride[4];
} lq_tensor;

/* ABI version (LQ_ABI_VERSION) of the loaded library. */
int lq_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* lq_last_error(void);

/*
 * Diagnostic switches, for tests and experiments (no counterpart in the reference). FORCE_*
 * sends every call of a kernel family to its general kernel; REQUIRE_* makes a call that would
 * take the general kernel fail with LQ_ERR_INVALID_ARG instead (a test's proof that a case runs
 * the fast kernel). The library reads them once from the environment variables of the same
 * names (set to anything but "" or "0") when it is loaded; afterwards only lq_set_diagnostics
 * changes them. The switches are process-wide: set them between calls, not while another thread
 * launches.
 */
enum {
  LQ_DIAG_ATTN_FORCE_GENERIC = 1u << 0,
  LQ_DIAG_ATTN_REQUIRE_FAST = 1u << 1,
  LQ_DIAG_PREFILL_FORCE_GENERIC = 1u << 2,
  LQ_DIAG_PREFILL_REQUIRE_MFMA = 1u << 3,
  LQ_DIAG_MX_FORCE_GENERIC = 1u << 4,
  LQ_DIAG_MX_REQUIRE_ROWS = 1u << 5,
  LQ_DIAG_SSM_FORCE_GENERIC = 1u << 6,
  LQ_DIAG_SSM_REQUIRE_ROWS = 1u << 7,
  /* split-K partials merged inside the fast attention kernel by each (batch, KV head)'s last
   * workgroup instead of by a second launch; off by default: slower at batch 1 (ctx 16384: 17.5
   * against 10.4 + 4.4 us of kernel time) and at batch 8, ctx 2072, 0.7 us faster at batch 8,
   * ctx 16384 */
  LQ_DIAG_ATTN_FOLD_MERGE = 1u << 8,
  LQ_DIAG_ALL = (1u << 9) - 1
};

/* The current LQ_DIAG_* bits. */
uint32_t lq_diagnostics(void);

/* Replaces the LQ_DIAG_* bits (unknown bits are dropped); returns the previous ones. */
uint32_t lq_set_diagnostics(uint32_t flags);

/*
 * INT4 pack of new K or V tokens into the packed cache.
 * Replaces the launch of _pack_int4_kv_kernel (reference hybrid_quant/int4_8b_attention.py:32-111,
 * launched twice by _pack_kv_into_cache at :477-514).
 *   x         [B, Hkv, q_len, D]  f32/f16/bf16, any strides
 *   packed    [B, Hkv, cap, D/2]  u8   (byte p holds d=2p in the low nibble, d=2p+1 in the high)
 *   scale     [B, Hkv, cap, D/g]  f32
 *   positions [q_len]             i64  cache row written for each new token
 * Per group of g values: scale = max(absmax/7, 1e-8); q = clamp(rint(x/scale), -8, 7).
 * Rows outside [0, cap) are skipped (the caller grows the cache first).
 */
int lq_int4_pack_kv(const lq_tensor* x, const lq_tensor* packed, const lq_tensor* scale,
                    const lq_tensor* positions, int group_size, void* stream);

/*
 * lq_int4_pack_kv for a layer's K and V in one launch (the same arguments and checks, applied to
 * (k, k_packed, k_scale) and (v, v_packed, v_scale) with shared positions).
 * No counterpart in the reference: it replaces the pair of _pack_int4_kv_kernel launches that
 * _pack_kv_into_cache makes (hybrid_quant/int4_8b_attention.py:487-514) with one.
 */
int lq_int4_pack_kv_pair(const lq_tensor* k, const lq_tensor* v, const lq_tensor* k_packed,
                         const lq_tensor* v_packed, const lq_tensor* k_scale,
                         const lq_tensor* v_scale, const lq_tensor* positions, int group_size,
                         void* stream);

/*
 * Workspace bytes that lq_int4_decode_attention needs for this shape (0 if none).
 * No counterpart in the reference (its decode kernel has no split-K); it sizes the split-K
 * partials of the kernel below. A workspace (256-byte aligned) starts with
 * LQ_DECODE_ATTENTION_COUNTER_BYTES of arrival counters, which must be zero before the workspace
 * is first used (e.g. allocate it zeroed); every call leaves them zero again, so a workspace can be
 * reused across calls of any shape, in order on one stream, and under HIP graph replay. (A call
 * that does not run to completion, e.g. one whose kernel is aborted, can leave them non-zero.)
 */
#define LQ_DECODE_ATTENTION_COUNTER_BYTES (64u << 10)
size_t lq_int4_decode_attention_workspace(int64_t batch, int64_t n_q_heads, int64_t n_kv_heads,
                                          int64_t head_dim, int64_t seq_len, int group_size);

/*
 * q_len = 1 GQA attention over the packed INT4 cache.
 * Replaces the launch of _int4_decode_attention_kernel (reference
 * hybrid_quant/int4_8b_attention.py:254-402, launched by _decode_attention at :518-566).
 *   q         [B, Hq, 1, D] or [B, Hq, D]   f32/f16/bf16
 *   k_packed, v_packed [B, Hkv, cap, D/2] u8;  k_scale, v_scale [B, Hkv, cap, D/g] f32
 *   mask      NULL or [B, 1, 1, Lm] f32 additive bias (only batch and key strides are used;
 *             keys at or beyond Lm get -inf, as in the reference)
 *   out       [B, Hq, D]   f32/f16/bf16
 * Keys [0, seq_len) are attended; q head h reads KV head h / num_key_value_groups.
 * Scores use exp2 with scale log2(e)/sqrt(D); softmax and accumulation are fp32.
 */
int lq_int4_decode_attention(const lq_tensor* q, const lq_tensor* k_packed,
                             const lq_tensor* v_packed, const lq_tensor* k_scale,
                             const lq_tensor* v_scale, const lq_tensor* mask, const lq_tensor* out,
                             int64_t seq_len, int num_key_value_groups, int group_size,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step of an attention layer: lq_int4_pack_kv_pair of the new token's k_new, v_new
 * [B, Hkv, 1, D] (f32/f16/bf16, any strides) into cache row seq_len - 1, then
 * lq_int4_decode_attention over keys [0, seq_len) -- the same checks, the same cache bytes and
 * the same output as those two calls. On the MFMA path (bf16 q, head_dim 128, group 32/64/128)
 * it is one launch: the wave that attends to key seq_len - 1 packs the token, writes it to the
 * cache and uses its own bytes for that key; elsewhere the two kernels run in turn. The workspace
 * is sized by lq_int4_decode_attention_workspace.
 * Replaces the decode branch of the reference's patched forward, _pack_kv_into_cache followed by
 * _decode_attention (reference hybrid_quant/int4_8b_attention.py:678-690; the kernels at :32-111
 * and :254-402).
 */
int lq_int4_decode_attention_pack(const lq_tensor* q, const lq_tensor* k_new,
                                  const lq_tensor* v_new, const lq_tensor* k_packed,
                                  const lq_tensor* v_packed, const lq_tensor* k_scale,
                                  const lq_tensor* v_scale, const lq_tensor* mask,
                                  const lq_tensor* out, int64_t seq_len, int num_key_value_groups,
                                  int group_size, void* workspace, size_t workspace_bytes,
                                  void* stream);

/*
 * lq_int4_decode_attention without a workspace: the same validation, kernels and results, with
 * the split-K partials in a static per-device buffer inside the library
 * (LQ_DECODE_ATTENTION_NOALLOC_SCRATCH_BYTES, 8 MiB on every GPU the library runs on, held until
 * the process ends). At 32 query / 8 KV heads and head_dim 128 any batch and context needs at
 * most 2 MiB of it; rarer shapes that need more (16 query heads per KV head, or head_dim 512, at
 * some batch sizes) get LQ_ERR_WORKSPACE (lq_int4_decode_attention_workspace gives the size a
 * shape needs). Calls no allocating routine.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Every call on one GPU shares that GPU's buffer; it keeps the last call's partials, and its
 * arrival counters (zero when the library loads) are left zero by every call: calls that overlap
 * on one GPU -- on different streams, or from
 * different host threads -- race and must be serialized by the caller; calls in order on one
 * stream are safe. The buffer is on the device that runs `stream`. The first call on a device
 * resolves the buffer's device address (hipGetSymbolAddress); make that call outside any HIP
 * graph capture (a warm-up call before capturing), after which captured calls only launch.
 */
#define LQ_DECODE_ATTENTION_NOALLOC_SCRATCH_BYTES (8u << 20)
int lq_int4_decode_attention_noalloc(const lq_tensor* q, const lq_tensor* k_packed,
                                     const lq_tensor* v_packed, const lq_tensor* k_scale,
                                     const lq_tensor* v_scale, const lq_tensor* mask,
                                     const lq_tensor* out, int64_t seq_len,
                                     int num_key_value_groups, int group_size, void* stream);

/*
 * Causal INT4 prefill attention over the packed cache: query position t of q [B, Hq, L, D]
 * attends to cache rows 0 .. t of KV head h / num_key_value_groups, scores (q . k) *
 * log2(e)/sqrt(D) in an exp2-domain softmax; out [B, Hq, L, D] (f32/bf16/f16). Replaces
 * _int4_prefill_attention_kernel and its launcher _prefill_attention (reference
 * hybrid_quant/int4_8b_attention.py:114-251, 594-625). Requires L <= capacity; any strides on
 * q and out; no workspace. MFMA path for head_dim 128, group 32/64/128 and bf16 q with
 * contiguous cache rows; a generic path otherwise.
 */
int lq_int4_prefill_attention(const lq_tensor* q, const lq_tensor* k_packed,
                              const lq_tensor* v_packed, const lq_tensor* k_scale,
                              const lq_tensor* v_scale, const lq_tensor* out,
                              int num_key_value_groups, int group_size, void* stream);

/*
 * MX state layouts. Every MX entry point takes either layout and tells them apart by the shapes
 * of q_state and micro_exp (N = 16 * shared_exp.shape[3]):
 *   reference layout (hybrid_quant/mamba_state_8b_kernel.py:11-25, 575-598):
 *     q_state [B,H,P,N] i8 (one byte per mantissa, also for MX4), shared_exp [B,H,P,N/16] u8
 *     (biased, 127 = 2^0), micro_exp [B,H,P,N/2] u8 (0/1 per pair);
 *   compact layout (no reference counterpart; same values, 2.5x (MX4) or 1.4x (MX8) fewer bytes):
 *     q_state [B,H,P,N] i8 for MX8, or [B,H,P,N/2] u8 for MX4 with element 2j in the low nibble
 *     of byte j and 2j+1 in the high (two's complement); shared_exp as above; micro_exp
 *     [B,H,P,N/16] u8 with bit k of byte b = the micro-exponent of pair k of block b.
 *   Nibble mantissas hold MX4 only (LQ_ERR_INVALID_ARG otherwise). Results are bit-identical in
 *   both layouts.
 *
 * MX block encode of a float state [B, H, P, N] (N % 16 == 0) into either layout.
 * format_bits 8 -> mantissa max 63, 4 -> 7. With LQ_ROUND_NEAREST_EVEN this replaces
 * _quantize_initial_state_mx (reference hybrid_quant/mamba_state_8b_kernel.py:547-572); the
 * other modes run the writeback encoder of :168-222 / :494-544 on a given state.
 *   uniform    [B,H,P,N] f32, required for LQ_ROUND_SR_UNIFORM, else NULL
 *   seed, rng_offset: counter of LQ_ROUND_SR_COUNTER and LQ_ROUND_SR_PHILOX (element (b,h,p,n)
 *   draws counter rng_offset + ((b*H + h)*P + p)*N + n)
 */
int lq_mx_encode(const lq_tensor* state, const lq_tensor* q_state, const lq_tensor* shared_exp,
                 const lq_tensor* micro_exp, int format_bits, int round_mode,
                 const lq_tensor* uniform, uint64_t seed, uint64_t rng_offset, void* stream);

/*
 * Dequantize an MX state: out[b,h,p,n] = q * 2^(shared_exp - 127 + micro_exp) (f32/bf16 out).
 * No kernel of its own in the reference (its update kernels decode inline at
 * hybrid_quant/mamba_state_8b_kernel.py:132 and :322); used to read a state back.
 */
int lq_mx_decode(const lq_tensor* q_state, const lq_tensor* shared_exp,
                 const lq_tensor* micro_exp, const lq_tensor* out, void* stream);

/*
 * Fused Mamba2 selective-state update over an MX8/MX4 state, in place:
 *   h  = q * 2^(e - 127 + micro)
 *   dt = dt (+ dt_bias); dt = softplus(dt) if dt_softplus (x <= 20 ? log(1+e^x) : x)
 *   h' = h * exp(A * dt) + (B * dt) * x;   y = sum_n h' * C (+ x * D) (* z)
 *   re-encode h' (format_bits 8 or 4) with round_mode, write y to out.
 * Replaces _state_update_requant_mx8_row_kernel (reference
 * hybrid_quant/mamba_state_8b_kernel.py:33-222) for MX8 and the pair
 * _state_update_mx8_kernel + _requantize_mx4_kernel (:225-443, :494-544) for MX4, as dispatched
 * by mx_state_selective_update (:601-721). One pass: no fp32 temporary state.
 *   x [B,H,P]; dt [B,H,P]; dt_bias NULL or [H,P]; A [H,P,N] f32; B, C [B,G,N] with H % G == 0;
 *   D NULL or [H,P]; z NULL or [B,H,P]; out [B,H,P]. Any strides (0 allowed) on these.
 *   q_state/shared_exp/micro_exp: innermost dimension contiguous.
 */
int lq_mx_state_update(const lq_tensor* q_state, const lq_tensor* shared_exp,
                       const lq_tensor* micro_exp, const lq_tensor* x, const lq_tensor* dt,
                       const lq_tensor* dt_bias, const lq_tensor* A, const lq_tensor* B,
                       const lq_tensor* C, const lq_tensor* D, const lq_tensor* z,
                       const lq_tensor* out, int format_bits, int dt_softplus, int round_mode,
                       const lq_tensor* uniform, uint64_t seed, uint64_t rng_offset, void* stream);

/*
 * lq_mx_state_update with the counter offset's step on the device: the same arguments and
 * results, with LQ_ROUND_SR_COUNTER's and LQ_ROUND_SR_PHILOX's offset
 * rng_offset + step[0] * B*H*P*N, where step is an int64 [1] tensor on the device that the
 * kernel reads when it runs (the reference's offsets
 * step*B*H*P*N with the step counter on the device; other rounding modes ignore it). A caller that
 * captures an update in a HIP graph and advances step inside the graph (e.g. a captured add of 1)
 * draws fresh values on every replay; with the host offset the draws of the capture would repeat.
 * No counterpart in the reference (its step counter is a host integer, baked into every Triton
 * launch, hybrid_quant/mamba_state_8b_kernel.py:659, 716).
 */
int lq_mx_state_update_device_step(const lq_tensor* q_state, const lq_tensor* shared_exp,
                                   const lq_tensor* micro_exp, const lq_tensor* x,
                                   const lq_tensor* dt, const lq_tensor* dt_bias,
                                   const lq_tensor* A, const lq_tensor* B, const lq_tensor* C,
                                   const lq_tensor* D, const lq_tensor* z, const lq_tensor* out,
                                   int format_bits, int dt_softplus, int round_mode,
                                   const lq_tensor* uniform, uint64_t seed, uint64_t rng_offset,
                                   const lq_tensor* step, void* stream);

/*
 * Selective-state update of an unquantized (bf16, fp16 or fp32) Mamba2 state, in place:
 *   dt = dt (+ dt_bias); dt = softplus(dt) if dt_softplus (x <= 20 ? log(1+e^x) : x)
 *   h' = h * exp(A * dt) + (B * dt) * x  (fp32, one fma per element, stored back with RNE)
 *   y  = sum_n h' * C (+ x * D);  y *= z * sigmoid(z) when z is given
 * Replaces mamba-ssm 2.3.2.post1's selective_state_update, which the reference calls for every
 * layer whose state is not registered for the MX kernel (the `original` fallback of
 * hybrid_quant/mamba_state_8b_kernel.py:738-747) and which is the bf16-state baseline of its
 * state experiments. Shapes as lq_mx_state_update with state [B,H,P,N] in place of the MX
 * tensors; every tensor may have any strides (0 allowed), the state a 16-byte aligned contiguous
 * last dimension for vector access.
 */
int lq_selective_state_update(const lq_tensor* state, const lq_tensor* x, const lq_tensor* dt,
                              const lq_tensor* dt_bias, const lq_tensor* A, const lq_tensor* B,
                              const lq_tensor* C, const lq_tensor* D, const lq_tensor* z,
                              const lq_tensor* out, int dt_softplus, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LAYER_QUANT_H_ */
