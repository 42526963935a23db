/* leatmi: the C ABI of the MI355X (gfx950) kernels for leat's quantized-weight linear layers.
 *
 * Every entry point is asynchronous on the caller's HIP stream (`stream`, a hipStream_t, or NULL
 * for the null stream), allocates nothing, keeps no state between calls and does not synchronise.
 * All pointers are device pointers the caller owns. Weights are GGUF blocks exactly as stored:
 * a (rows, cols) matrix is rows * cols / elements blocks, row after row (leat/quant.py:234-251).
 * Return value: 0, or -1 with a message in leat_last_error() (bad type, shape or pointer, or a
 * failed launch). Reference paths below are in alkinun/leat. An output may be its call's residual
 * buffer (a residual stream updated in place); it must not overlap the call's other inputs.
 */
#ifndef LEATMI_H
#define LEATMI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGMLType ids of the storage types these kernels read (leat/quant.py:14-46) */
#define LEAT_Q8_0 8
#define LEAT_Q4_K 12
#define LEAT_Q6_K 14

/* GLU kinds (leat/kernels/common.py:299-321) */
#define LEAT_GLU_SILU 0
#define LEAT_GLU_GELU 1
#define LEAT_GLU_OAI 2

/* The message of the last failed call on this thread. */
const char *leat_last_error(void);
/* ABI revision of this header, and the device architecture the kernels are built for. */
int leat_abi_version(void);
const char *leat_target(void);

/* Replaces leat/kernels/quantize.py:92-109 quantize_q8(x, norm, rows). x (rows, n) f32, n a
 * multiple of 32; norm_weight (n) f32 or NULL for no RMSNorm, eps its epsilon. Writes q
 * (rows * n / 4) int32 words of four int8 values, d and s (rows * n / 32) f32: d = max|x|/127,
 * q = roundf(x / d), s = d * sum(q) per group of 32. */
int leat_quantize_q8(const float *x, int rows, int n, const float *norm_weight, float eps,
                     int32_t *q, float *d, float *s, void *stream);

/* Replaces the custom kernel of leat/kernels/matvec.py:362-380 matvecs() for one matrix
 * (_matvec_kernel, :306-321): out[t * rows + r] = W[r] . x[t] (+ residual[t * rows + r] if
 * residual is not NULL), x given as quantize_q8's (xq, xd, xs) for `tokens` rows of `cols`
 * values. tokens: 1..8, or up to 16 where the matrix-core decode kernels take the shape (16-byte
 * aligned rows and matrices). cols: a multiple of 256 for Q4_K/Q6_K, of 64 for Q8_0. */
int leat_matvec(int type, const void *w, int rows, int cols, const int32_t *xq, const float *xd,
                const float *xs, int tokens, const float *residual, float *out, void *stream);

/* Replaces the loop over ws of leat/kernels/matvec.py:372-380 (matvecs(x, *ws) sharing one
 * quantization): `count` matrices of the same cols; consecutive ones of one type run in one
 * launch (up to 4). outs[i] receives tokens * rows[i] values, token-major. */
int leat_matvecs(int count, const int *types, const void *const *ws, const int *rows, int cols,
                 const int32_t *xq, const float *xd, const float *xs, int tokens,
                 float *const *outs, void *stream);

/* Replaces leat/kernels/matvec.py:383-395 swiglu() (_swiglu_kernel, :324-337):
 * out[t * rows + r] = glu(kind)(gate[r] . x[t], up[r] . x[t]), gate and up of one type and shape,
 * both in one kernel. */
int leat_glu_matvec(int type, const void *gate, const void *up, int rows, int cols,
                    const int32_t *xq, const float *xd, const float *xs, int tokens, int kind,
                    float *out, void *stream);

/* leat_glu_matvec that also writes leat_quantize_q8 of its outputs, (tokens, rows) as
 * (tokens * rows / 4) words and (tokens * rows / 32) scales and sums: the down product's input, as
 * leat's feed_forward quantizes it (leat/ops.py:41-55). rows a multiple of 32. For 1..2 tokens and
 * for 3..8 tokens of 16-byte aligned Q4_K the GLU kernel writes them itself; otherwise a quantize
 * launch follows it. out is required. */
int leat_glu_matvec_q8(int type, const void *gate, const void *up, int rows, int cols,
                       const int32_t *xq, const float *xd, const float *xs, int tokens, int kind,
                       float *out, int32_t *hq, float *hd, float *hs, void *stream);

/* Replaces the whole of leat/kernels/matvec.py:362-380 matvecs(x, *ws, norm) for one or two
 * tokens: quantize_q8 of x (after RMSNorm with norm_weight and eps when norm_weight is not NULL)
 * and the products, in one launch. Each workgroup quantizes x itself with leat_quantize_q8's
 * arithmetic, so the outputs are bit-identical to leat_quantize_q8 followed by leat_matvecs.
 * x (tokens, cols) f32, 16-byte aligned; 1 to 4 matrices of one type, Q4_K (cols a multiple of
 * 256, at most 8192), Q8_0 (a multiple of 64, at most 8192) or Q6_K (a multiple of 512, at most
 * 8192); tokens 1 or 2. */
int leat_matvecs_f32(int count, const int *types, const void *const *ws, const int *rows, int cols,
                     const float *x, int tokens, const float *norm_weight, float eps,
                     float *const *outs, void *stream);

/* The same for one matrix with an optional residual (leat/kernels/matvec.py:362-380 with
 * residual): out[t * rows + r] = W[r] . q8(x[t]) (+ residual[t * rows + r]). */
int leat_matvec_f32(int type, const void *w, int rows, int cols, const float *x, int tokens,
                    const float *norm_weight, float eps, const float *residual, float *out,
                    void *stream);

/* Replaces leat/kernels/matvec.py:383-395 swiglu(x, gate, up, norm, kind) for one or two tokens
 * in one launch, x quantized inside as in leat_matvecs_f32. out (tokens * rows f32) may be NULL
 * when hq is given. When hq, hd and hs are given (rows a multiple of 32) the kernel also writes
 * leat_quantize_q8 of its outputs, (tokens, rows) as (tokens * rows / 4) words and
 * (tokens * rows / 32) scales and sums: the down product's input, as leat's feed_forward
 * quantizes it (leat/ops.py:41-55), without another launch. */
int leat_glu_matvec_f32(int type, const void *gate, const void *up, int rows, int cols,
                        const float *x, int tokens, const float *norm_weight, float eps, int kind,
                        float *out, int32_t *hq, float *hd, float *hs, void *stream);

/* Replaces the LEAT_KERNELS=ref linear layer, leat/ops.py:35-38 (x @ w.dequant().T with f32
 * activations, not quantized): out[t * rows + r] = W[r] . x[t] (+ residual), W decoded in
 * ggml's operation order, f32 sums. x (tokens, cols) f32; tokens 1..8 or 16. */
int leat_matvec_f32x(int type, const void *w, int rows, int cols, const float *x, int tokens,
                     const float *residual, float *out, void *stream);

/* Replaces leat/quant.py:246-251 QTensor.dequant() for the types above: n_blocks blocks to
 * n_blocks * elements f32, bit-identical to ggml's dequantize_row_* (no fused multiply-add). */
int leat_dequantize(int type, const void *blocks, int64_t n_blocks, float *out, void *stream);

/* Parity probe with no counterpart in leat (whose kernels keep these sums in registers,
 * leat/kernels/matvec.py:114-181): the exact int32 sums of weight and activation integers per
 * scale span, computed by the matvec kernels' own decode: groups of 32 for Q4_K (nibbles 0..15)
 * and Q8_0, halves of 16 for Q6_K (q - 32). out[(t * rows + r) * spans + span], spans = cols/32
 * (Q4_K, Q8_0) or cols/16 (Q6_K). */
int leat_group_dots(int type, const void *w, int rows, int cols, const int32_t *xq, int tokens,
                    int32_t *out, void *stream);

/* The bytes of workspace leat_matmul (gated = 0) or leat_glu_matmul / leat_glu_matmul_q8
 * (gated = 1) split a product of this shape into, on the current device; 0 when it runs unsplit.
 * Replaces the parts buffer of leat/kernels/matmul.py:1005-1010 (_products with a schedule). */
int64_t leat_matmul_workspace(int type, int rows, int cols, int tokens, int gated);

/* Replaces the custom kernel of leat/kernels/matmul.py:1051-1066 matmuls() (_matmul_kernel,
 * :631-841, with its schedule and fixup :856-964) for many tokens: out[t * rows + r] = W[r] . x[t]
 * (+ residual), x as quantize_q8's (xq, xd, xs) for `tokens` rows of `cols`. int8 products per
 * group of 32 on matrix cores, scaled per group in f32. Up to 16 tokens (leat's FEW_TOKENS) take
 * 32-row by 16-token tiles; more take 64-token tiles, and when those are fewer than the GPU runs
 * at once each tile's K steps are split over several workgroups, their sums left in `workspace`
 * (leat_matmul_workspace bytes; with less, or NULL, the product runs unsplit) and added by a
 * fixup launch in a fixed order. cols a multiple of 256 (512 for Q6_K); weights 4-byte (Q4_K:
 * 16-byte) and xq 16-byte aligned. */
int leat_matmul(int type, const void *w, int rows, int cols, const int32_t *xq, const float *xd,
                const float *xs, int tokens, const float *residual, float *out, void *workspace,
                int64_t workspace_bytes, void *stream);

/* No counterpart in leat: leat_matmul for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc). A split product's partial sums go to
 * a file-scope device array of 8 MiB on each GPU instead of a caller workspace; products whose
 * split needs more (leat_matmul_workspace) return -1. Calls on one GPU share its array: calls that
 * overlap on one GPU race, calls in one stream order do not. Allocates nothing. */
int leat_matmul_noalloc(int type, const void *w, int rows, int cols, const int32_t *xq,
                        const float *xd, const float *xs, int tokens, const float *residual,
                        float *out, void *stream);

/* Replaces the gated product of leat/kernels/matmul.py:1069-1081 feed_forward() (_products with
 * gated=True): out[t * rows + r] = glu(kind)(gate[r] . x[t], up[r] . x[t]), gate and up in one
 * kernel. Same shape, tile and workspace rules as leat_matmul. */
int leat_glu_matmul(int type, const void *gate, const void *up, int rows, int cols,
                    const int32_t *xq, const float *xd, const float *xs, int tokens, int kind,
                    float *out, void *workspace, int64_t workspace_bytes, void *stream);

/* The same and, for the down product of leat/kernels/matmul.py:1069-1081 feed_forward(), the
 * quantize_q8 of its outputs: hq (tokens * rows / 4 words), hd and hs (tokens * rows / 32),
 * bit-identical to leat_quantize_q8 of out. rows a multiple of 32. For Q4_K past 16 tokens the
 * GLU kernel writes them itself, and out may be NULL (no f32 outputs); otherwise out is required
 * and a quantize launch follows. */
int leat_glu_matmul_q8(int type, const void *gate, const void *up, int rows, int cols,
                       const int32_t *xq, const float *xd, const float *xs, int tokens, int kind,
                       float *out, int32_t *hq, float *hd, float *hs, void *workspace,
                       int64_t workspace_bytes, void *stream);

/* Replaces leat/kernels/experts.py:163-172 route() (_route_kernel, :132-160): for each of `tokens`
 * rows of scores (tokens, experts) f32, the `used` best experts by repeated argmax (ties to the
 * lower id; -inf and NaN count as the least finite score) as ids (tokens * used) int32, and the
 * softmax of their scores as weights (tokens * used) f32. experts <= 256, used <= 64. */
int leat_route(const float *scores, int tokens, int experts, int used, int32_t *ids, float *weights,
               void *stream);

/* Replaces leat/kernels/experts.py:110-124 scores() (_scores_kernel, :44-64): a mixture's router
 * scores in f32, out[t * experts + e] = (sum_i x[t,i] * norm_weight[i] * router[e,i]) /
 * sqrt(mean(x[t]^2) + eps), for x (tokens, dim) f32 and an F32 router (experts, dim). dim a
 * multiple of 4; x, norm_weight and router 16-byte aligned. */
int leat_scores(const float *x, int tokens, int dim, const float *norm_weight, float eps,
                const float *router, int experts, float *out, void *stream);

/* Replaces the expert kernel of leat/kernels/experts.py:341-359 (_experts_swiglu_kernel,
 * :209-238): out[p * rows + r] = glu(kind)(gate[e] row r . x[p / used] + gate_bias[e * rows + r],
 * up[e] row r . x[p / used] + up_bias[e * rows + r]) for pairs p < pairs, e = ids[p], x as
 * quantize_q8's (xq, xd, xs). gate and up: stacks of `experts` (rows, cols) matrices; up NULL:
 * gate stacks both, each expert's gate rows before its up rows. Biases may be NULL. Each chosen
 * expert's rows are read once for all the pairs routed to it. */
int leat_experts_glu(int type, const void *gate, const void *up, int experts, int rows, int cols,
                     const int32_t *xq, const float *xd, const float *xs, const int32_t *ids, int pairs,
                     int used, const float *gate_bias, const float *up_bias, int kind, float *out,
                     void *stream);

/* Replaces the first four steps of a decode mixture, leat/kernels/experts.py:341-359 (route,
 * quantize_q8 of rms_norm(x), experts_swiglu) and the quantize_q8 of its hidden rows that
 * leat_experts_down consumes, in one launch: routes `tokens` (1..8) rows of scores (tokens,
 * experts) f32 as leat_route (writing ids and weights, tokens * used), quantizes x (tokens, cols)
 * f32 after RMSNorm with norm_weight and eps (NULL: none) as leat_quantize_q8, and computes
 * out[p * rows + r] as leat_experts_glu; out may be NULL. hq, hd, hs receive leat_quantize_q8 of
 * those pairs * rows values (rows a multiple of 32). Limits: experts <= 256, used <= 64; rows of
 * Q4_K (cols a multiple of 256), Q6_K (of 512) or Q8_0 (of 64) of at most 8192 weights; x and
 * norm_weight 16-byte aligned. An expert chosen by k tokens is read k times (one workgroup a pair:
 * faster at 8 tokens than sharing its rows). */
int leat_experts_glu_f32(int type, const void *gate, const void *up, int experts, int rows, int cols,
                         const float *x, int tokens, const float *norm_weight, float eps,
                         const float *scores, int used, const float *gate_bias, const float *up_bias,
                         int kind, int32_t *ids, float *weights, float *out, int32_t *hq, float *hd,
                         float *hs, void *stream);

/* Replaces the down kernel of leat/kernels/experts.py:360-371 (_experts_down_kernel, :241-270):
 * out[t * rows + r] = sum over slots s < used of weights[p] * scales[e] * (w[e] row r . h[p]
 * + bias[e * rows + r]) (+ residual[t * rows + r]), p = t * used + s, e = ids[p]; h the pairs'
 * hidden states as quantize_q8's (hq, hd, hs), tokens * used rows of cols. w: a stack of
 * `experts` (rows, cols) matrices. scales, bias and residual may be NULL. used 1..64. */
int leat_experts_down(int type, const void *w, int experts, int rows, int cols, const int32_t *hq,
                      const float *hd, const float *hs, const int32_t *ids, const float *weights,
                      int tokens, int used, const float *scales, const float *bias,
                      const float *residual, float *out, void *stream);

/* ---------------------------------------------------------------- the decode step around them */

/* Replaces leat/ops.py:166-178 embedding(tokens, w): out[t, :] = row ids[t] of W decoded to f32 as
 * leat_dequantize decodes it (ids outside 0..rows-1 give zeros). ids is a device array. */
int leat_embedding(int type, const void *w, int rows, int cols, const int32_t *ids, int tokens,
                   float *out, void *stream);

/* Replaces leat/kernels/attention.py:656-782 rotate() for heads without biases or norms: each
 * token's q (tokens, heads, dim) and k (tokens, kv_heads, dim) turned by RoPE over the first
 * `rotated` dimensions (pairs of adjacent dimensions, or with `halves` dimensions i and
 * i + rotated / 2), by the angles of the token's position in cos and sin (cache_positions,
 * rotated / 2) f32; q to q_out (heads, tokens, dim) f32, and k with v (tokens, kv_heads, dim)
 * stored as f16 in the cache (2, cache_slots, kv_heads, cache_positions, dim) at the token's
 * slot and position. slots and positions are device arrays; a token whose slot or position
 * lies outside the cache stores nothing. */
int leat_rotate(const float *q, const float *k, const float *v, int tokens, int heads, int kv_heads,
                int dim, const float *cos, const float *sin, int rotated, int halves,
                const int32_t *slots, const int32_t *positions, float *q_out, void *cache,
                int cache_slots, int cache_positions, void *stream);

/* Replaces leat/kernels/matvec.py:362-380 matvecs(x, q, k, v, norm) followed by
 * leat/kernels/attention.py:656-782 rotate() for 1..2 tokens, in one launch: x (tokens, cols) f32
 * RMS-normalized with norm_weight and quantized as leat_matvecs_f32 does, the q (heads * dim), k
 * and v (kv_heads * dim rows) products, then q and k turned by RoPE over the first `rotated`
 * dimensions of each head (pairs of adjacent dimensions, by the angles of the token's position
 * in cos and sin), q to q_out (heads, tokens, dim) f32 and k with v stored as f16 in the cache
 * (2, cache_slots, kv_heads, cache_positions, dim) at the token's slot and position: bit for bit
 * what leat_matvecs_f32 then leat_rotate (halves = 0) give. dim a multiple of 16; the three
 * matrices of one type, rows as leat_matvecs_f32 takes them. A token whose slot or position
 * lies outside the cache stores nothing. */
int leat_qkv_rotate_f32(int type, const void *wq, const void *wk, const void *wv, int heads,
                        int kv_heads, int dim, int cols, const float *x, int tokens,
                        const float *norm_weight, float eps, const float *cos, const float *sin,
                        int rotated, const int32_t *slots, const int32_t *positions, float *q_out,
                        void *cache, int cache_slots, int cache_positions, void *stream);

/* The workspace bytes leat_attention needs for `rows` rows of `heads` heads and rows of at most
 * max_length keys. */
int64_t leat_attention_workspace(int rows, int heads, int max_length);

/* Replaces leat/kernels/attention.py:226-279 attention() (FlashDecoding): for each row (a query
 * token), out[row, h * dim ..] = softmax over keys 0 .. lengths[row] - 1 of slot slots[row] of
 * (q[h, row] . key * scale) times the values, kv head h / (heads / kv_heads); q (heads, rows, dim)
 * f32 as leat_rotate writes it, the f16 cache as leat_rotate fills it, out (rows, heads * dim)
 * f32. Scores, weights and sums in f32. dim 128; 1, 2, 4 or 8 query heads a kv head; slots and
 * lengths device arrays, every length at most max_length (which sizes the launch). */
int leat_attention(const float *q, const void *cache, int cache_slots, int kv_heads,
                   int cache_positions, int dim, int rows, int heads, const int32_t *slots,
                   const int32_t *lengths, int max_length, float scale, float *workspace,
                   int64_t workspace_bytes, float *out, void *stream);

/* leat_attention that also writes the q8 of its output (no counterpart in leat, whose o product
 * quantizes the attention output itself, leat/kernels/matvec.py:362-380 through
 * leat/kernels/quantize.py:92-109): hq, hd, hs exactly what leat_quantize_q8 writes for the rows
 * of heads * dim values in out, for the q8-input product that follows (leat_matvec). hq 4-byte
 * aligned. */
int leat_attention_q8(const float *q, const void *cache, int cache_slots, int kv_heads,
                      int cache_positions, int dim, int rows, int heads, const int32_t *slots,
                      const int32_t *lengths, int max_length, float scale, float *workspace,
                      int64_t workspace_bytes, float *out, int32_t *hq, float *hd, float *hs,
                      void *stream);

/* The workspace bytes leat_argmax needs for `rows` rows. */
int64_t leat_argmax_workspace(int rows);

/* Replaces leat/kernels/argmax.py:14-59 argmax(x): out[row] = the index of the largest value of
 * row `row` of x (rows, n) f32, the lowest index among equal values; NaN is never chosen. */
int leat_argmax(const float *x, int rows, int n, void *workspace, int64_t workspace_bytes,
                int32_t *out, void *stream);

/* Measurement probes, with no counterpart in leat: the rates this GPU reaches, reported beside the
 * published peaks that the benchmark's rooflines divide by.
 * leat_probe_read: streams `bytes` (whole 16-byte chunks, 16-byte aligned) with 16-byte loads and
 * leaves in sink[g], for each of `workgroups` workgroups, its share of the sum of every 32-bit word
 * modulo 2^32 (the sink values add up to the whole sum).
 * leat_probe_mfma_i8: `workgroups` workgroups of 4 waves, each wave running `iters` rounds of 4
 * independent v_mfma_i32_32x32x32_i8 on all-ones operands (65,536 ops each); sink[4 g + w] =
 * 128 * iters. */
int leat_probe_read(const void *data, int64_t bytes, uint32_t *sink, int workgroups, void *stream);
int leat_probe_mfma_i8(int iters, int workgroups, int32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LEATMI_H */
