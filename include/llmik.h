/*
 * llmik.h — C ABI of the gfx950 decode-step hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), enqueues its kernels asynchronously on that stream and
 * returns an llmik_status. Nothing here allocates device memory: outputs
 * and the optional workspace are supplied by the caller. No torch types
 * appear in any signature.
 *
 * Each function cites the reference operator it replaces: the torch op in
 * bindings/extension.cpp of bundle-adjuster/llm-inference-kernels and the
 * CUDA launcher behind it.
 *
 * Tensor conventions (row-major, contiguous, 16-byte aligned base pointers):
 *   fp16 tensors are IEEE binary16 bit patterns (uint16_t);
 *   int8 codes are int8_t; packed int4 is one byte per two codes with the
 *   even channel in the low nibble; W4 weights are uint32 words holding
 *   8 codes along K (bits 4i..4i+3 = K position 8*k_pack + i).
 *
 * Workspace contract (attention and W4A16): query the size with the
 * matching *_workspace_size function. The first LLMIK_WORKSPACE_COUNTER_BYTES
 * bytes of every workspace hold completion counters: they must be zero
 * before the first use, every successful call leaves them zero again, and
 * no entry point writes anything else there. One zero-filled buffer can
 * therefore be reused by consecutive calls of any of these entry points on
 * one stream. Calls that share a workspace must not run concurrently.
 */
#ifndef LLMIK_H
#define LLMIK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMIK_API __attribute__((visibility("default")))

typedef int llmik_status;
#define LLMIK_OK 0
/* Negative codes are argument/usage errors detected before any launch;
 * positive codes are hipError_t values returned by the HIP runtime. */
#define LLMIK_ERR_INVALID (-1)
#define LLMIK_ERR_UNSUPPORTED (-2)
#define LLMIK_ERR_WORKSPACE (-3)
#define LLMIK_ERR_ALIGNMENT (-4)

/* Size of the zero-initialised counter region at the start of a workspace. */
#define LLMIK_WORKSPACE_COUNTER_BYTES 16384

/* Message for the last error raised on the calling thread ("" if none). */
LLMIK_API const char* llmik_last_error(void);
/* ABI version; bumped on any signature change. */
LLMIK_API int llmik_abi_version(void);

/* ---------------------------------------------------------------- attention
 * Workspace bytes needed by the decode-attention entry points for this
 * shape on the current device (0 means none needed; pass NULL).
 */
LLMIK_API size_t llmik_attention_workspace_size(int batch, int n_heads, int n_kv_heads,
                                                int seqlen, int head_dim);

/*
 * fp16-KV split-K GQA decode attention.
 * Replaces: decode_attention op (bindings/extension.cpp:26-83) and
 *   launch_decode_attention_splitk / decode_attention_n_splits
 *   (kernels/attention/fused_attention.cuh:32-41,
 *   kernels/attention/fused_attention_splitk.cu:64-66,233-250); also serves
 *   decode_attention_v3 (bindings/extension.cpp:89-115; launch_decode_attention,
 *   kernels/attention/fused_attention.cuh:17-20, fused_attention.cu:110-119)
 *   with seqlen == kv_buf_len, since the result semantics are identical.
 *   q   [batch, n_heads, head_dim] fp16
 *   k,v [batch, n_kv_heads, kv_buf_len, head_dim] fp16; positions
 *       [0, seqlen) are read (seqlen <= kv_buf_len)
 *   out [batch, n_heads, head_dim] fp16
 * head_dim must be 128; n_heads must be a multiple of n_kv_heads.
 */
LLMIK_API llmik_status llmik_decode_attention_f16(
    const void* q, const void* k, const void* v, void* out,
    int batch, int n_heads, int n_kv_heads, int seqlen, int head_dim, int kv_buf_len,
    float softmax_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * INT8 per-token KV decode attention with fused dequantisation.
 * Replaces: decode_attention_int8 op (bindings/extension.cpp:152-194) and
 *   launch_decode_attention_int8 (kernels/attention/fused_attention.cuh:54-60,
 *   kernels/attention/fused_attention_int8.cu:109-122).
 *   k_q,v_q         [batch, n_kv_heads, kv_buf_len, head_dim] int8
 *   k_scale,v_scale [batch, n_kv_heads, kv_buf_len] fp16
 * The reference op has no live-length argument; seqlen == kv_buf_len
 * reproduces it. seqlen < kv_buf_len reads a preallocated cache in place.
 */
LLMIK_API llmik_status llmik_decode_attention_int8(
    const void* q, const void* k_q, const void* k_scale, const void* v_q, const void* v_scale,
    void* out, int batch, int n_heads, int n_kv_heads, int seqlen, int head_dim, int kv_buf_len,
    float softmax_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * INT4 KIVI KV decode attention (K per-channel groupwise, V per-token,
 * symmetric, packed) with fused dequantisation.
 * Replaces: decode_attention_int4 op (bindings/extension.cpp:269-314) and
 *   launch_decode_attention_int4 (kernels/attention/fused_attention.cuh:73-80,
 *   kernels/attention/fused_attention_int4.cu:120-135).
 *   k_q,v_q [batch, n_kv_heads, kv_buf_len, head_dim/2] int8 (packed int4)
 *   k_scale [batch, n_kv_heads, n_groups, head_dim] fp16; token t uses
 *           group t / group_size (needs n_groups >= ceil(seqlen/group_size))
 *   v_scale [batch, n_kv_heads, kv_buf_len] fp16
 */
LLMIK_API llmik_status llmik_decode_attention_int4(
    const void* q, const void* k_q, const void* k_scale, const void* v_q, const void* v_scale,
    void* out, int batch, int n_heads, int n_kv_heads, int seqlen, int head_dim, int kv_buf_len,
    int group_size, int n_groups, float softmax_scale, void* workspace, size_t workspace_bytes,
    void* stream);

/*
 * The same fp16 decode attention with no workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The split-K counters and partials live in a static device
 * array of LLMIK_NOALLOC_SCRATCH_BYTES per device (held until the process
 * ends); a call whose plan needs more (llmik_attention_workspace_size)
 * returns LLMIK_ERR_WORKSPACE. It calls no allocator. All calls on one device
 * share that array: calls that overlap on a device race, so issue them in
 * one stream order. Results are bit-identical to llmik_decode_attention_f16.
 */
#define LLMIK_NOALLOC_SCRATCH_BYTES (2u << 20)
LLMIK_API llmik_status llmik_decode_attention_f16_noalloc(
    const void* q, const void* k, const void* v, void* out,
    int batch, int n_heads, int n_kv_heads, int seqlen, int head_dim, int kv_buf_len,
    float softmax_scale, void* stream);

/* --------------------------------------------------------------- KV writers
 * Bit-exact symmetric quantisers: scale = max(absmax/qmax, 1e-8) in fp32
 * with IEEE division, q = clamp(round_half_even(x / scale), -qmax, qmax),
 * scale stored as fp16 (round to nearest even). This is
 * reference/kv_cache_ref.py applied to x.float().
 */

/*
 * INT8 per-token quantisation (qmax 127).
 * Replaces: quantize_per_token op (bindings/extension.cpp:120-146) and
 *   launch_quantize_per_token (kernels/kv_cache/kv_compress.cuh:19-22,
 *   kernels/kv_cache/kv_compress.cu:69-79).
 *   x [batch, n_kv_heads, seqlen, head_dim] fp16 -> q int8 same shape,
 *   scale [batch, n_kv_heads, seqlen] fp16.
 */
LLMIK_API llmik_status llmik_quantize_per_token_int8(
    const void* x, void* q, void* scale, int batch, int n_kv_heads, int seqlen, int head_dim,
    void* stream);

/*
 * INT4 K quantisation, per channel, grouped along the sequence (qmax 7).
 * Replaces: quantize_k_per_channel_groupwise_int4 op
 *   (bindings/extension.cpp:200-229) and its launcher
 *   (kernels/kv_cache/kv_compress.cuh:35-39, kv_compress.cu:159-170).
 *   x [batch, n_kv_heads, seqlen, head_dim] fp16 ->
 *   q [batch, n_kv_heads, seqlen, head_dim/2] packed int4,
 *   scale [batch, n_kv_heads, ceil(seqlen/group_size), head_dim] fp16.
 *   A short final group uses only its real tokens.
 */
LLMIK_API llmik_status llmik_quantize_k_per_channel_groupwise_int4(
    const void* x, void* q, void* scale, int batch, int n_kv_heads, int seqlen, int head_dim,
    int group_size, void* stream);

/*
 * INT4 V quantisation, per token (qmax 7).
 * Replaces: quantize_v_per_token_int4 op (bindings/extension.cpp:235-261)
 *   and its launcher (kernels/kv_cache/kv_compress.cuh:45-48,
 *   kv_compress.cu:219-228).
 *   x [batch, n_kv_heads, seqlen, head_dim] fp16 ->
 *   q [batch, n_kv_heads, seqlen, head_dim/2] packed int4,
 *   scale [batch, n_kv_heads, seqlen] fp16.
 */
LLMIK_API llmik_status llmik_quantize_v_per_token_int4(
    const void* x, void* q, void* scale, int batch, int n_kv_heads, int seqlen, int head_dim,
    void* stream);

/* ------------------------------------------------- in-place KV-cache writers
 * The same quantisers writing into a preallocated cache at a token offset,
 * so a growing cache is appended to in place instead of being rebuilt.
 * Replaces: the torch.cat of freshly quantised chunks onto the whole packed
 *   cache in Int4KIVICache.append_only / get_quantized_for_attention
 *   (integration/kv_int4_cache.py:119-144,184-206), which calls the
 *   writers above on each chunk; the quantiser arithmetic is theirs.
 *   x           [batch, n_kv_heads, x_len, head_dim] fp16; tokens [0, n_tok)
 *               of each (batch, kv_head) row are quantised
 *   q_cache     [batch, n_kv_heads, cache_len, head_dim] int8 (INT8) or
 *               [batch, n_kv_heads, cache_len, head_dim/2] packed int4
 *   scale_cache [batch, n_kv_heads, cache_len] fp16 (per token) or
 *               [batch, n_kv_heads, ceil(cache_len/group_size), head_dim]
 *               fp16 (K per channel, group-wise)
 * Token t is written to cache position offset + t (offset + n_tok <=
 * cache_len); nothing else in the cache is touched. The codes and scales
 * are bit-identical to the out-of-place writer applied to those tokens.
 */
LLMIK_API llmik_status llmik_quantize_per_token_int8_into(const void* x, int x_len, void* q_cache,
                                                          void* scale_cache, int batch,
                                                          int n_kv_heads, int n_tok, int head_dim,
                                                          int cache_len, int offset, void* stream);
LLMIK_API llmik_status llmik_quantize_v_per_token_int4_into(const void* x, int x_len, void* q_cache,
                                                            void* scale_cache, int batch,
                                                            int n_kv_heads, int n_tok, int head_dim,
                                                            int cache_len, int offset, void* stream);
/* offset must be a multiple of group_size: tokens [offset, offset + n_tok)
 * form ceil(n_tok / group_size) groups, the last one possibly partial (its
 * scale uses only its real tokens, as the out-of-place writer does). */
LLMIK_API llmik_status llmik_quantize_k_per_channel_groupwise_int4_into(
    const void* x, int x_len, void* q_cache, void* scale_cache, int batch, int n_kv_heads,
    int n_tok, int head_dim, int cache_len, int offset, int group_size, void* stream);

/* One decode-step token appended to a KIVI INT4 cache in one launch: the
 * three launches of Int4KIVICache.append for one token (V per token at
 * position `length`; K into the open group's fp16 tokens and the open group
 * re-quantised into its codes and scale slot), the same stored bits.
 * Replaces, for one token, the reference's per-append re-quantise and
 * torch.cat (integration/kv_int4_cache.py:104-144,168-206).
 *   k, v     [batch, n_kv_heads, k_len / v_len, 128] fp16; token 0 is appended
 *   k_open   [batch, n_kv_heads, group_size, 128] fp16: the open group's tokens
 *            0 .. length % group_size - 1; the new token is written after them
 *   k_q, v_q [batch, n_kv_heads, max_len, 64] packed int4
 *   k_scale  [batch, n_kv_heads, ceil(max_len / group_size), 128] fp16
 *   v_scale  [batch, n_kv_heads, max_len] fp16
 * group_size <= 128; length < max_len. */
LLMIK_API llmik_status llmik_kivi_append_token_int4(
    const void* k, int k_len, const void* v, int v_len, void* k_open, void* k_q, void* k_scale, void* v_q,
    void* v_scale, int batch, int n_kv_heads, int head_dim, int max_len, int group_size, int length,
    void* stream);

/* -------------------------------------------------------------------- W4A16
 * out[M, N] = act[M, K] @ dequant(W)[K, N], W[k, n] = q[k, n] * scale[k/g, n],
 * fp32 accumulation.
 *   act           [M, K] fp16
 *   weight_packed [K/8, N] uint32 (int4 along K)
 *   scale         [K/group_size, N] fp16
 * group_size must be a positive multiple of 8 dividing K. act and
 * weight_packed need 16-byte, scale 8-byte and out 4-byte alignment; a
 * 16-byte aligned out lets the 64 x 128-tile M > 16 matrix-core GEMM store
 * 8 / 16 bytes at a time (otherwise it stores one value at a time, as the
 * 256 x 128-tile GEMM that serves M >= 256 with many tiles always does).
 */
LLMIK_API size_t llmik_w4a16_workspace_size(int M, int N, int K, int group_size);

/*
 * Replaces: w4a16_gemm op (bindings/extension.cpp:322-376) and
 *   launch_w4a16_gemm / launch_w4a16_gemm_splitk / w4a16_n_splits
 *   (kernels/quant/quant_matmul.cuh:30-44, quant_matmul.cu:642-652,778-856).
 *   out [M, N] fp16.
 */
LLMIK_API llmik_status llmik_w4a16_gemm(
    const void* act, const void* weight_packed, const void* scale, void* out,
    int M, int N, int K, int group_size, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Same kernels with an fp32 output (the accumulator before fp16 rounding).
 * No reference counterpart: it exists so the 2e-3 max-abs gate against an
 * fp32-accumulated oracle can be checked without fp16 output rounding.
 */
LLMIK_API llmik_status llmik_w4a16_gemm_f32out(
    const void* act, const void* weight_packed, const void* scale, void* out_f32,
    int M, int N, int K, int group_size, void* workspace, size_t workspace_bytes, void* stream);

/*
 * A gate|up projection and its SwiGLU in one launch (the decode step's MLP;
 * no single counterpart in the reference, which runs the gate and up
 * QuantizedLinear projections and silu(gate) * up as separate ops,
 * integration/prealloc_cache.py:129-130). weight_packed [K/8, N] / scale
 * [K/g, N] hold the gate and up weights with their columns interleaved in
 * 64-column tiles: tile t is gate columns 32t .. 32t+31, then up columns
 * 32t .. 32t+31. out [M, N/2] fp16 gets fp16(silu(g) * u) of the
 * fp16-rounded products g = (act @ W)[:, 64t + j], u = (act @ W)[:, 64t + 32 + j]
 * at column 32t + j: the bits of llmik_w4a16_gemm on the concatenated
 * weight followed by llmik_silu_mul_halves when both run the streaming
 * GEMV. Needs 1 <= M <= 16, N % 64 == 0, K % 32 == 0 and a power-of-two
 * group_size >= 32 (LLMIK_ERR_UNSUPPORTED otherwise); the workspace is
 * llmik_w4a16_swiglu_workspace_size(M, N, K, group_size) bytes, with the
 * rules of llmik_w4a16_gemm.
 */
LLMIK_API size_t llmik_w4a16_swiglu_workspace_size(int M, int N, int K, int group_size);
LLMIK_API llmik_status llmik_w4a16_gemm_swiglu(const void* act, const void* weight_packed,
                                               const void* scale, void* out, int M, int N, int K,
                                               int group_size, void* workspace, size_t workspace_bytes,
                                               void* stream);

/*
 * The decode step's q|k|v projection, its rope and the cache append in one
 * launch (head_dim 128): llmik_w4a16_gemm over the concatenated q | k | v
 * weight followed by llmik_rope_qkv_append_f16, with the same bits when both
 * run the streaming GEMV. No single counterpart in the reference, which runs
 * the q, k and v QuantizedLinear projections, rope of q and k and the cache
 * update as separate ops (integration/prealloc_cache.py:42-110,132-133).
 * weight_packed [K/8, N] / scale [K/g, N], N = (n_heads + 2 n_kv_heads) 128,
 * hold the concatenated weight with each head's two 64-dimension halves
 * interleaved in 32-column blocks: the head's columns are dimensions 0..31,
 * 64..95, 32..63, 96..127. cos / sin are the position's [128] fp16 rotary
 * rows; q_out [batch, n_heads, 128] gets the roped q, slot `pos` of k_cache /
 * v_cache [batch, n_kv_heads, max_len, 128] the roped k and v. Needs
 * 1 <= batch <= 16, K % 32 == 0 and a power-of-two group_size >= 32
 * (LLMIK_ERR_UNSUPPORTED otherwise), pos < max_len; the alignment rules of
 * llmik_w4a16_gemm with q_out as its out, 2 bytes for cos, sin and the
 * caches; workspace of llmik_w4a16_qkv_rope_workspace_size(...) bytes, with
 * the rules of llmik_w4a16_gemm.
 */
LLMIK_API size_t llmik_w4a16_qkv_rope_workspace_size(int batch, int n_heads, int n_kv_heads, int K,
                                                     int group_size);
LLMIK_API llmik_status llmik_w4a16_gemm_qkv_rope_f16(
    const void* act, const void* weight_packed, const void* scale, const void* cos, const void* sin,
    void* q_out, void* k_cache, void* v_cache, int batch, int K, int group_size, int n_heads,
    int n_kv_heads, int max_len, int pos, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Plan knobs of the W4A16 entry points, for measurement and tests (no
 * reference counterpart). stream_mode: 1 forces the streaming GEMV wherever
 * the shape allows, 0 disables it, -1 restores the size rule; stream_splits
 * > 0 forces its K split count, <= 0 restores the planner's. The library
 * reads the initial values once, when it loads, from LLMIK_W4A16_STREAM and
 * LLMIK_W4A16_STREAM_SPLITS. Not synchronised with calls in flight on other
 * threads.
 */
LLMIK_API void llmik_w4a16_set_plan_override(int stream_mode, int stream_splits);

/*
 * Plan knob of the fp16 attention entry points, for measurement and tests (no
 * reference counterpart). f16_half_tiles: 1 runs every fp16 call on the MFMA
 * path with 16-token tiles, 0 with 32-token tiles, -1 restores the rule (16-
 * token tiles for at least 32 (batch, kv head, head chunk) slabs, a
 * workgroup count that is a multiple of the CU count, and at least two
 * 32-token tiles per wave unless the workgroups have 4 waves). Not
 * synchronised with calls in flight on other threads.
 */
LLMIK_API void llmik_attention_set_plan_override(int f16_half_tiles);

/*
 * Materialise fp16 W[k, n] = fp16(q[k, n] * scale[k/g, n]).
 * Replaces: w4a16_dequantize op (bindings/extension.cpp:382-403) and
 *   launch_w4a16_dequantize (kernels/quant/quant_matmul.cuh:58-60;
 *   kernels/quant/quant_matmul.cu:629-638). out [K, N] fp16.
 */
LLMIK_API llmik_status llmik_w4a16_dequantize(
    const void* weight_packed, const void* scale, void* out, int K, int N, int group_size,
    void* stream);

/*
 * Symmetric INT4 group-wise weight quantisation on the GPU, bit-exact to the
 * reference's host-side torch function.
 * Replaces: quantize_weights_int4_groupwise (reference/quant_matmul_ref.py:39-88),
 *   which the reference runs with torch ops when a layer is converted
 *   (integration/w4a16_patch.py:78-84) and in its tests
 *   (tests/test_quant.py:265-267).
 *   W         [K, N] fp16 (w_fp16 != 0) or fp32
 *   q         [K, N] int8 codes in [-7, 7], or NULL
 *   packed    [K/8, N] int32 (pack_int4_along_k of q), or NULL; needs K and
 *             group_size to be multiples of 8
 *   scale     [ceil(K/group_size), N] in W's dtype, or NULL
 *   scale_f16 [ceil(K/group_size), N] fp16 (scale rounded to fp16, the
 *             convention of integration/w4a16_patch.py:84), or NULL
 * scale = max(absmax_group |W| / 7, 1e-8) evaluated in W's dtype (fp16:
 * the quotient is rounded to fp16 and the floor is fp16(1e-8) = 0); codes
 * are clamp(rint(fp32 W / fp32 scale), -7, 7) with true division and
 * half-to-even rounding, NaN -> 0; a short last group uses its real rows.
 */
LLMIK_API llmik_status llmik_quantize_weights_int4_groupwise(
    const void* W, int w_fp16, int K, int N, int group_size, void* q, void* packed, void* scale,
    void* scale_f16, void* stream);

/*
 * Replaces: pack_int4_along_k (reference/quant_matmul_ref.py:140-165).
 *   q [K, N] int8 -> packed [K/8, N] int32, bits 4i..4i+3 of word (kp, n) =
 *   q[8 kp + i, n] & 0xF. K must be a multiple of 8.
 */
LLMIK_API llmik_status llmik_pack_int4_along_k(const void* q, int K, int N, void* packed,
                                               void* stream);

/* ------------------------------------------------------ fused elementwise ops */

/*
 * out[r, :] = fp16(x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * weight), fp32 math.
 * Replaces: rmsnorm op (bindings/extension.cpp:408-424) and launch_rmsnorm
 *   (kernels/fused/fused_ops.cuh:9-11, kernels/fused/fused_ops.cu:96-100).
 */
LLMIK_API llmik_status llmik_rmsnorm(const void* x, const void* weight, void* out, int rows,
                                     int hidden, float eps, void* stream);

/*
 * out = fp16(silu(gate) * up), elementwise over n values.
 * Replaces: silu_mul op (bindings/extension.cpp:427-441) and launch_silu_mul
 *   (kernels/fused/fused_ops.cuh:13-14, kernels/fused/fused_ops.cu:102-107).
 */
LLMIK_API llmik_status llmik_silu_mul(const void* gate, const void* up, void* out, long n,
                                      void* stream);

/*
 * out = x * cos + rotate_half(x) * sin, x [B, H, S, D], cos/sin [B, S, D].
 * Replaces: rope op (bindings/extension.cpp:446-473) and launch_rope
 *   (kernels/fused/fused_ops.cuh:17-18, kernels/fused/fused_ops.cu:88-94).
 */
LLMIK_API llmik_status llmik_rope(const void* x, const void* cos, const void* sin, void* out,
                                  int B, int H, int S, int D, void* stream);

/* --------------------------------------------------- decode-step merged ops
 * Consecutive ops of the reference's patched decode step
 * (integration/prealloc_cache.py:61-76,113-144: the in-place cache write,
 * RMSNorm, SwiGLU, RoPE) merged into one launch each. Each computes what the ops it
 * replaces compute, with the same roundings; no single reference function
 * corresponds to them. */

/*
 * qkv [batch, n_heads + 2 n_kv_heads, head_dim] fp16: one token's fused
 * q|k|v projection. q_out [batch, n_heads, head_dim] = rope(q);
 * k_cache[b, h, pos, :] = rope(k[b, h]); v_cache[b, h, pos, :] = v[b, h];
 * caches [batch, n_kv_heads, max_len, head_dim]. cos / sin: the position's
 * [head_dim] row of the rotary tables, as llmik_rope applies it.
 * Replaces: rope of q and k (rope_fwd, integration/prealloc_cache.py:132-133)
 *   and the cache-slot writes of PreallocCache.update (:61-76).
 */
LLMIK_API llmik_status llmik_rope_qkv_append_f16(const void* qkv, const void* cos, const void* sin,
                                                 void* q_out, void* k_cache, void* v_cache, int batch,
                                                 int n_heads, int n_kv_heads, int head_dim, int max_len,
                                                 int pos, void* stream);

/*
 * h_out = fp16(x + residual) and out = llmik_rmsnorm(h_out, weight, eps),
 * [rows, hidden] fp16, hidden % 8 == 0 and hidden <= 8192.
 * Replaces: a decoder layer's residual add (transformers' LlamaDecoderLayer)
 *   and the RMSNorm after it (rms_fwd, integration/prealloc_cache.py:126-127).
 */
LLMIK_API llmik_status llmik_add_rmsnorm(const void* x, const void* residual, const void* weight,
                                         void* h_out, void* out, int rows, int hidden, float eps,
                                         void* stream);

/*
 * out[r, c] = fp16(silu(gate_up[r, c]) * gate_up[r, cols + c]) over a fused
 * gate|up projection gate_up [rows, 2 cols] fp16; cols % 8 == 0.
 * Replaces: llmik_silu_mul on the gate and up projections' separate outputs
 *   (mlp_fwd, integration/prealloc_cache.py:129-130).
 */
LLMIK_API llmik_status llmik_silu_mul_halves(const void* gate_up, void* out, long rows, int cols,
                                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LLMIK_H */
