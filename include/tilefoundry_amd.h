/*
 * tilefoundry_amd -- C ABI of the MI355X (gfx950) per-layer LLM kernels.
 *
 * Conventions for every entry point:
 *   - tensors are raw device pointers; bf16 tensors are passed as `void*` and
 *     hold IEEE bfloat16 bit patterns; f32 as `float*`; ids / positions as
 *     int32 / int64 device pointers;
 *   - all tensors are dense row-major with the shape stated in the comment;
 *   - nothing allocates and nothing synchronises: work is enqueued on `stream`
 *     and every entry point may be recorded into a HIP graph;
 *   - positions, write slots and context lengths that change from step to step
 *     are read on the device (int32 tensors), never baked into a launch;
 *   - the return value is a tfa_status; on failure tfa_last_error() names the
 *     entry point and the reason.
 *
 * Reference citations are to jingchangshi/TileFoundry (paths relative to the
 * repository root).
 */
#ifndef TILEFOUNDRY_AMD_H_
#define TILEFOUNDRY_AMD_H_

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TFA_ABI_VERSION 1

enum tfa_status {
  TFA_OK = 0,
  TFA_ERR_NULL = 1,      /* a required pointer is null */
  TFA_ERR_SHAPE = 2,     /* a dimension is outside what the kernel supports */
  TFA_ERR_ALIGN = 3,     /* a pointer is not 16-byte aligned */
  TFA_ERR_CAPACITY = 4,  /* a length exceeds a buffer's capacity */
  TFA_ERR_ARG = 5,       /* an argument value is invalid (mode, eps, ...) */
  TFA_ERR_LAUNCH = 6     /* the HIP runtime refused the launch */
};

int tfa_abi_version(void);
const char* tfa_status_string(int status);
/* Message of the last failing call on this thread ("" if none). */
const char* tfa_last_error(void);

/* ------------------------------------------------------------------ norms */

/* y[r,:] = rmsnorm(x[r,:]) over rows x hidden.
 * mode 0: y = bf16(bf16(x*rsqrt(mean x^2 + eps)) * gamma)    (Qwen3, MiniCPM3)
 * mode 1: y = bf16(x*rsqrt(mean x^2 + eps) * (1 + gamma))    (Qwen3.5 prefill)
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:58-79 (rms_norm, one
 * row) and examples/qwen3_8_27b_prefill-tilelang/kernels/elementwise.py:21-68
 * (rmsnorm_kernel, many rows). hidden % 8 == 0, hidden <= 8192. */
int tfa_rms_norm(const void* x, const void* gamma, void* y, int64_t rows, int64_t hidden,
                 float eps, int mode, hipStream_t stream);

/* y[r,:] = bf16(bf16(bf16(x*rsqrt(mean x^2 + eps)) * gamma) / divisor), the divide
 * correctly rounded: MiniCPM3's final norm followed by the head's division by
 * logits_scaling (a divide, since 1/10 is not a bf16 number). divisor != 0.
 * Replaces: examples/minicpm3_4b-cutedsl/model.py:367-392 (MiniCPM3_4B.final_rms_norm and
 * the divide of lm_head), kernels/reference_ops.py:78-84 (lm_head_gemv's divide). */
int tfa_rms_norm_div(const void* x, const void* gamma, void* y, int64_t rows, int64_t hidden, float eps,
                     float divisor, hipStream_t stream);

/* Fused residual add + RMSNorm over rows x hidden:
 *   residual_out = bf16(x + residual);  y = rmsnorm(residual_out) (mode as above).
 * residual_out may alias residual and y may alias x.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:82-116 (resid_rms_norm)
 * generalised to rows; HIR `h1 = hidden + attn_out` then the norm
 * (examples/qwen3_1_7b-tilelang/ref_src/model.py:263,226-228). */
int tfa_add_rms_norm(const void* x, const void* residual, const void* gamma, void* y,
                     void* residual_out, int64_t rows, int64_t hidden, float eps, int mode,
                     hipStream_t stream);

/* One row: h_out = bf16(a + bf16(sum_s partials[s,:])); xn = rmsnorm(h_out) (mode 0).
 * partials is f32 [splits, hidden].
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:82-116 (resid_rms_norm). */
int tfa_resid_rms_norm_partials(const void* a, const float* partials, int64_t splits,
                                const void* gamma, void* h_out, void* xn, int64_t hidden,
                                float eps, hipStream_t stream);

/* ------------------------------------------------- decode GEMVs, W [N, K] */
/* Weights are row-major [N, K] = (out, in), the checkpoint's own layout.
 * K % 32 == 0, K <= 8192; x / h / gamma / w 16-byte aligned. */

/* y[n] = sum_k x[k] w[n,k]; y is f32 (out_f32 != 0) or bf16.
 * Replaces: examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:57-58 (gemv),
 * examples/minicpm3_4b-cutedsl/kernels/cute_gemv.py:430-495. */
int tfa_gemv(const void* x, const void* w, void* y, int64_t n, int64_t k, int out_f32,
             hipStream_t stream);

/* y = bf16(rmsnorm(h) . w^T) (norm mode 0). Replaces
 * examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:46-48 (rmsnorm_gemv),
 * cute_gemv.py:246-286 (NORM_GEMV). */
int tfa_rmsnorm_gemv(const void* h, const void* gamma, float eps, const void* w, void* y,
                     int64_t n, int64_t k, hipStream_t stream);

/* The same product left in f32 (y[n] = rmsnorm(h) . w[n], no landing): one
 * sequence's [q_a | kv_a] projection as the single split-K partial the MLA
 * prep lands in bf16. Replaces: examples/minicpm3_4b-cutedsl/kernels/cute_gemv.py:246-286
 * (NORM_GEMV over the fused q_a / kv_a weights, runtime_model.py's first launch of a layer). */
int tfa_rmsnorm_gemv_f32(const void* h, const void* gamma, float eps, const void* w, float* y,
                         int64_t n, int64_t k, hipStream_t stream);

/* One sequence's MLA prep fused into the q_b GEMV: part = [q_a (q_lora) |
 * kv_c (256) | k_rope (32)] f32, the single split-K partial that
 * tfa_rmsnorm_gemv_f32 leaves; every block lands q_a in bf16, takes its LoRA
 * norm with gamma_q_a (summed in tfa_mla_prep's order, so q_n is bit-equal)
 * and writes q_part[n] = q_n . w_q_b[n] (f32, w_q_b [n, q_lora]); block 0 also
 * writes latent_cache[pos[0]] and rope_cache[pos[0]] exactly as tfa_mla_prep
 * does (caches [cap, 256] / [cap, 32] bf16; a pos outside [0, cap) or the
 * rope table sets *err = 6 and skips them). q_lora a multiple of 32, <= 1024.
 * Replaces: examples/minicpm3_4b-cutedsl/model.py:220-250 (steps 1-4 of
 * mla_attention at one sequence) and kernels/cute_gemv.py:246-286 (NORM_GEMV
 * of q_b over the normalised q_a). */
int tfa_mla_prep_q_gemv(const float* part, int64_t q_lora, const void* gamma_q_a, const void* gamma_kv_a,
                        float eps, const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos,
                        void* latent_cache, void* rope_cache, int64_t cap, const void* w_q_b, float* q_part,
                        int64_t n, int* err, hipStream_t stream);

/* y[n] = bf16(residual[n] + bf16(x.w[n])), or with alpha (bf16 [1]):
 * y[n] = bf16(residual[n] + bf16(bf16(x.w[n]) * alpha)).  y may not alias residual.
 * Replaces: the residual adds of examples/qwen3_1_7b-tilelang/ref_src/model.py:263-265
 * (folded into o_proj / down_proj) and
 * examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:61-63 (gemv_residual). */
int tfa_gemv_residual(const void* x, const void* w, const void* residual, const void* alpha,
                      void* y, int64_t n, int64_t k, hipStream_t stream);

/* act[i] = bf16(bf16(silu(bf16 g_i)) * bf16 u_i) with (g_i, u_i) = rmsnorm(h) . (w_gu[2i], w_gu[2i+1]).
 * w_gu is [2*inter, K] with gate and up rows interleaved.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:210-257 (gemv_silu's prologue)
 * and :547-572 (silu_mul); HIR mlp examples/qwen3_1_7b-tilelang/ref_src/model.py:217-233. */
int tfa_rmsnorm_gemv_swiglu(const void* h, const void* gamma, float eps, const void* w_gu,
                            void* act, int64_t inter, int64_t k, hipStream_t stream);

/* The same SwiGLU with gate and up as two [inter, K] matrices (no interleaving):
 * act[i] = bf16(bf16(silu(bf16 g_i)) * bf16 u_i), g = rmsnorm(h) . w_gate^T,
 * u = rmsnorm(h) . w_up^T. Replaces
 * examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:66-70 (rmsnorm_gemv_swiglu)
 * and kernels/cute_gemv.py:352-425 (NORM_GEMV_SWIGLU). */
int tfa_rmsnorm_gemv_gate_up(const void* h, const void* gamma, float eps, const void* w_gate,
                             const void* w_up, void* act, int64_t inter, int64_t k,
                             hipStream_t stream);

/* Number of (value, index) block entries tfa_lm_head_argmax writes for `vocab`. */
int64_t tfa_lm_head_blocks(int64_t vocab);

/* Head: logits = rmsnorm(h) . w^T in f32 (gamma == NULL: h as is), plus each
 * block's best (max, lowest index) into block_val / block_idx
 * (tfa_lm_head_blocks(vocab) entries). w is [vocab, k] (the tied embedding table
 * serves as is). Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:260-321
 * (lm_head). */
int tfa_lm_head_argmax(const void* h, const void* gamma, float eps, const void* w, int64_t vocab,
                       int64_t k, float* logits, float* block_val, int* block_idx,
                       hipStream_t stream);

/* logits[n] = bf16(sum_k bf16(h[k] / divisor) w[n, k]) in bf16 (divisor != 0; a
 * correctly rounded f32 divide, not a reciprocal multiply). w is [vocab, k].
 * Replaces examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:78-84
 * (lm_head_gemv) and kernels/cute_gemv.py:500-531 (LM_HEAD). */
int tfa_lm_head_gemv(const void* h, const void* w, float divisor, void* logits, int64_t vocab,
                     int64_t k, hipStream_t stream);

/* Greedy pick + sample step on the device: best = argmax over the block
 * winners (lowest index on ties); sam[pos] = best; ids[0] = pos+1 < prompt_len ?
 * inp[pos+1] : best; pos += 1. inp / sam are int32 [nsteps].
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:591-637 (sample_step). */
int tfa_sample_step(const float* block_val, const int* block_idx, int64_t nblocks, const int* inp,
                    const int* prompt_len, int64_t* ids, int* pos, int* sam, int64_t nsteps,
                    int* err, hipStream_t stream);

/* act[r, i] = bf16(bf16(silu(bf16 g)) * bf16 u), g / u the sums over ks (<= 8)
 * split-K partials part[ks, rows, 2 * inter] (gate in [0, inter), up in
 * [inter, 2 inter)). Replaces examples/qwen3_1_7b-tilelang/fast/kernels.py:547-572
 * (silu_mul). */
int tfa_silu_mul(const float* part, int64_t ks, int64_t inter, int64_t rows, void* act,
                 hipStream_t stream);

/* out[r, :] = table[ids[r], :] (scaled == 0) or bf16(table[ids[r], :] * scale).
 * hidden % 8 == 0. An id outside [0, vocab) reads row 0 and sets err = 1.
 * Replaces examples/qwen3_1_7b-tilelang/fast/kernels.py:579-588 (embed) and
 * examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:72-76 (embed_scaled). */
int tfa_embed(const void* table, const int64_t* ids, int64_t vocab, int64_t hidden, int64_t rows,
              int scaled, float scale, void* out, int* err, hipStream_t stream);

/* Decode q|k|v projection: x = rmsnorm(h) (or rmsnorm(table[ids[0]]) when
 * table != NULL, the gathered row also written to h_copy); y = x . w_qkv^T with
 * w_qkv [(n_qk + n_v), hidden]; rows [0, n_qk) -> qk_out (bf16, raw: the head
 * norm and RoPE are applied by tfa_decode_attention), rows [n_qk, n_qk + n_v)
 * -> v_cache row wr[0] ([cap, n_v]). err (optional int32[1]) receives a nonzero
 * code if a device-resident index is out of range.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:58-79 + :123-145 +
 * :579-588 (rms_norm, gemv(qkv), embed) and the value write of :328-411. */
int tfa_decode_qkv(const void* h, const void* table, const int64_t* ids, int64_t vocab,
                   void* h_copy, const void* gamma_in, float eps, const void* w_qkv,
                   int64_t hidden, int64_t n_qk, int64_t n_v, void* qk_out, const int* wr,
                   void* v_cache, int64_t cap, int* err, hipStream_t stream);

/* Split-KV GQA decode attention (head_dim 128) for `batch` sequences, each with
 * its own cache [cap, hkv*128] (position-major; k_cache / v_cache are
 * [batch, cap, hkv*128]) attending its slots 0..wr[b]. Scores scaled by `scale`
 * in f32 after the dot; softmax in f32 per split of `split` (32, 64, 128 or 256)
 * slots; bf16 weights into P.V. Partials op [batch, cap/split, hq, 128],
 * mp / lp [batch, cap/split, hq]; splits past wr[b] are left untouched unless
 * `neutral` (then m = -1e30, l = 0, o = 0).
 * Prepared mode (gamma_q == NULL): q is the final query [batch, hq*128] and the
 * caches already hold slot wr. Fused mode: q is the raw [q | k] projection
 * [batch, (hq+hkv)*128] bf16 (the value row is already in v_cache), or -- when
 * qkv_part != NULL -- the raw [q | k | v] projection is the sum of part_ks f32
 * split-K partials [part_ks, batch, (hq+2hkv)*128]; each query head gets
 * Qwen3RMSNorm (gamma_q, eps_head) and rotate-half RoPE at pos[b] (cos / sin
 * [rope_rows, 128]); the new key gets the same with gamma_k and is written to
 * k_cache row wr[b] (and, from partials, the new value row to v_cache row wr[b]).
 * err (optional int32[1]): 4 = wr out of [0, cap) -- the reads are clamped to
 * slots 0..cap-1 and no cache row is written; 5 = pos out of [0, rope_rows).
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501 (attn_partial)
 * and :328-411 (qk_rope_cache). */
int tfa_decode_attention(const void* q, const float* qkv_part, int64_t part_ks,
                         const void* gamma_q, const void* gamma_k, float eps_head,
                         const void* cos_t, const void* sin_t, int64_t rope_rows, void* k_cache,
                         void* v_cache, const int* pos, const int* wr, int64_t batch, int64_t hq,
                         int64_t hkv, int64_t head_dim, int64_t cap, int64_t split, float scale,
                         float* op, float* mp, float* lp, int neutral, int* err,
                         hipStream_t stream);

/* One step of GQA decode attention with the query prep fused and no split:
 * one block per (sequence, kv head) over the whole context 0..wr[b]. From the
 * q|k|v split-K partials qkv_part [part_ks (<= 8), batch, (hq + 2 hkv) * 128]
 * f32 (each value landing in bf16): the query heads get Qwen3RMSNorm (gamma_q,
 * eps_head) + rotate-half RoPE at pos[b] (cos / sin [rope_rows, 128]), the key
 * the same with gamma_k and is written to k_cache row wr[b], the value row to
 * v_cache row wr[b] (caches [batch, cap, hkv * 128]). Then per query head
 * s = scale q.k, e = exp(s - max s) in f32, out[b, h*128 + d] =
 * bf16(sum bf16(e) v / sum e) -> out [batch, hq * 128] bf16. hq / hkv in
 * {1, 2, 4}; (cap + 64) * (hq / hkv) <= 32768. For batches whose sequences x kv
 * heads fill the device (the grid is hkv x batch blocks).
 * err: 4 = wr out of [0, cap) (the heads' output is zero), 5 = pos out of
 * [0, rope_rows).
 * Replaces, for one step: examples/qwen3_1_7b-tilelang/fast/kernels.py:328-411
 * (qk_rope_cache), :418-501 (attn_partial) and :504-540 (attn_combine). */
int tfa_decode_attention_seq(const float* qkv_part, int64_t part_ks, const void* gamma_q,
                             const void* gamma_k, float eps_head, const void* cos_t, const void* sin_t,
                             int64_t rope_rows, void* k_cache, void* v_cache, const int* pos, const int* wr,
                             int64_t batch, int64_t hq, int64_t hkv, int64_t head_dim, int64_t cap, float scale,
                             void* out, int* err, hipStream_t stream);

/* out[b, h*D + d] = bf16(sum_s op[b,s,h,d] e^(mp-M) / sum_s lp[b,s,h] e^(mp-M))
 * over all `splits`, or (wr != NULL) over the splits holding slots 0..wr[b].
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:504-540 (attn_combine). */
int tfa_attn_combine(const float* op, const float* mp, const float* lp, void* out, int64_t splits,
                     int64_t batch, int64_t hq, int64_t head_dim, const int* wr, int64_t split,
                     hipStream_t stream);

/* One sequence's split merge folded into the o_proj GEMV with its residual:
 * a = merge of op [splits, hq, 128] / mp / lp [splits, hq] exactly as
 * tfa_attn_combine (over the splits holding slots 0..wr[0] when wr != NULL),
 * y[r] = bf16(residual[r] + bf16(a . w_o[r])) for w_o [n, hq * 128] -- bit-identical
 * to tfa_attn_combine followed by tfa_gemv_residual, in one launch. attn_out
 * (nullable, bf16 [hq * 128]) receives a. hq a multiple of 4 in [4, 16];
 * splits <= 64; n <= 2560.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:154-207 (gemv_attn_combine)
 * with the residual add of examples/qwen3_1_7b-tilelang/ref_src/model.py:263. */
int tfa_attn_combine_gemv_residual(const float* op, const float* mp, const float* lp, int64_t splits, int64_t hq,
                                   int64_t head_dim, const int* wr, int64_t split, const void* w_o,
                                   const void* residual, void* y, int64_t n, void* attn_out, hipStream_t stream);

/* Reduce the q|k|v split-K partials qkv_part [part_ks (<= 8), batch,
 * (hq + 2 hkv) * 128] f32 (each value landing in bf16); per query head
 * Qwen3RMSNorm (gamma_q, eps_head) + rotate-half RoPE at pos[b] -> q_out
 * [batch, hq * 128]; the key head the same with gamma_k -> k_cache row wr[b];
 * the value head as is -> v_cache row wr[b] (caches [batch, cap, hkv * 128]).
 * err: 3 = wr out of [0, cap), 5 = pos out of [0, rope_rows).
 * Replaces examples/qwen3_1_7b-tilelang/fast/kernels.py:328-411 (qk_rope_cache). */
int tfa_qk_rope_cache(const float* qkv_part, int64_t part_ks, const void* gamma_q,
                      const void* gamma_k, float eps_head, const void* cos_t, const void* sin_t,
                      int64_t rope_rows, const int* pos, const int* wr, void* k_cache,
                      void* v_cache, int64_t cap, void* q_out, int64_t batch, int64_t hq,
                      int64_t hkv, int64_t head_dim, int* err, hipStream_t stream);

/* --------------------------------------------- batched decode (<= 32 rows) */

/* Groups of 16 weight rows: the per-token winner count of the argmax epilogue
 * for n rows. */
int64_t tfa_skinny_blocks(int64_t n);

/* Y = X[m, k] . W[n, k]^T for m <= 32 token rows on bf16 MFMA (f32 accumulate).
 * epilogue 0: f32 split-K partials part[ks, m, n] (sum over ks = Y);
 * epilogue 1 (ks = 1): SwiGLU over interleaved rows (2i, 2i+1) = (gate_i, up_i):
 *             act[m, n/2] = bf16(bf16(silu(bf16 g)) * bf16 u);
 * epilogue 2 (ks = 1): per token, each 16-row group's best (max, lowest index)
 *             into block_val / block_idx [m, tfa_skinny_blocks(n)], and the f32
 *             logits[m, n] when `logits` is not NULL;
 * epilogue 3 (ks = 1): as 2 with every logit landed in bf16 first (the winner
 *             among equal bf16 logits is the lowest index), for heads whose
 *             reference returns bf16 logits.
 * k % (256 * ks) == 0.
 * Replaces (batched): examples/qwen3_1_7b-tilelang/fast/kernels.py:123-145 (gemv),
 * :210-257 (gemv_silu), :260-321 (lm_head); epilogue 3 the greedy pick over
 * examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:78-84 (lm_head_gemv, bf16). */
int tfa_skinny_gemm(const void* x, const void* w, int64_t m, int64_t n, int64_t k, int64_t ks,
                    int epilogue, float* part, void* act, float* logits, float* block_val,
                    int* block_idx, hipStream_t stream);

/* Per token row: h = table[ids[r]] (table != NULL) or
 * h = bf16(h_in[r] + bf16(sum_s part[s, r, :])) (ks partials [ks, m, hidden]);
 * h_out[r] = h (may alias h_in); xn[r] = bf16(bf16(h * rsqrt(mean h^2 + eps)) * gamma).
 * Replaces (batched): examples/qwen3_1_7b-tilelang/fast/kernels.py:82-116
 * (resid_rms_norm) and :579-588 (embed). */
int tfa_rows_norm(const void* table, const int64_t* ids, int64_t vocab, const void* h_in,
                  const float* part, int64_t ks, void* h_out, const void* gamma, void* xn,
                  int64_t m, int64_t hidden, float eps, int* err, hipStream_t stream);

/* MiniCPM3's scaled residual followed by the next norm, per token row:
 * h = bf16(h_in[r] + bf16(bf16(sum_s part[s, r, :]) * alpha)), h_out[r] = h (may
 * alias h_in), xn[r] = bf16(bf16(h * rsqrt(mean h^2 + eps)) * gamma); alpha is
 * scale_depth / sqrt(layers). The rows_residual of one block fused with the norm
 * that opens the next.
 * Replaces: examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:63-65 (gemv_residual,
 * scaled) followed by :42-48 (rmsnorm), model.py:320-344 (decoder_layer's residuals). */
int tfa_rows_norm_scaled(const float* part, int64_t ks, const void* h_in, float alpha, void* h_out,
                         const void* gamma, void* xn, int64_t m, int64_t hidden, float eps, hipStream_t stream);

/* The batched o_proj with the residual add and the post-attention norm's sums
 * folded in: h_out[i, :] = bf16(res[i, :] + bf16(x[i, :] . w^T)) for m <= 32
 * token rows, x [m, k], w [n, k] (out, in), k a multiple of 256; and per
 * 32-row block b of w, ssq[b, i] = sum over the block's rows j of h_out[i, j]^2
 * (f32; tfa_skinny_residual_blocks(n) blocks). With
 * tfa_skinny_gemm_norm_swiglu it takes the place of tfa_skinny_gemm
 * (partials) + tfa_rows_norm: one launch fewer.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:82-116 (resid_rms_norm: its
 * residual add and the sum of squares) with the o_proj GEMV :123-145 before it. */
int64_t tfa_skinny_residual_blocks(int64_t n);
int tfa_skinny_gemm_residual(const void* x, const void* w, int64_t m, int64_t n, int64_t k, const void* res,
                             void* h_out, float* ssq, hipStream_t stream);

/* The batched gate|up GEMM + SwiGLU over the residual stream h [m, k] itself:
 * each token row is staged as xn = bf16(bf16(h * r) * gamma), r = 1 / sqrt(
 * sum_b ssq[b, i] / k + eps) (ssq [nssq <= 64, m] from tfa_skinny_gemm_residual,
 * summed in b order), then act = the SwiGLU epilogue of tfa_skinny_gemm
 * (epilogue 1) over interleaved gate|up rows, w [n, k], n even.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:82-116 (resid_rms_norm: the
 * norm) and :210-257 (gemv_silu's SwiGLU) around the gate|up GEMV. */
int tfa_skinny_gemm_norm_swiglu(const void* h, const void* w, int64_t m, int64_t n, int64_t k, const float* ssq,
                                int64_t nssq, const void* gamma, float eps, void* act, hipStream_t stream);

/* The greedy step for `batch` sequences: per sequence b, best = argmax over
 * block_val[b, :] (lowest index on ties); sam[b, pos[b]] = best;
 * ids[b] = pos[b]+1 < prompt_len[b] ? inp[b, pos[b]+1] : best; pos[b] += 1.
 * inp / sam are [batch, nsteps].
 * Replaces (batched): examples/qwen3_1_7b-tilelang/fast/kernels.py:591-637. */
int tfa_batch_sample_step(const float* block_val, const int* block_idx, int64_t nblocks,
                          int64_t batch, const int* inp, const int* prompt_len, int64_t* ids,
                          int* pos, int* sam, int64_t nsteps, int* err, hipStream_t stream);

/* The sampling step for `batch` sequences (vocab <= 81920): per sequence b,
 * probabilities softmax(logits[b] / T) (logits [batch, vocab] f32); ranked in
 * descending order (ties in index order), a token is kept while the mass ranked
 * before it is below top_p; one draw from the kept mass with a counter-based
 * generator of (seed[0], b, pos[b]) -- reproducible, and a different stream per
 * sequence and position. params = {T, top_p} (device f32[2], T > 0, top_p > 0).
 * Then sam[b, pos[b]] = the draw; ids[b] = pos[b]+1 < prompt_len[b] ?
 * inp[b, pos[b]+1] : the draw; pos[b] += 1 (inp / sam [batch, nsteps]).
 * err (optional): 2 = pos out of [0, nsteps).
 * Replaces: examples/minicpm3_4b-cutedsl/run.py:29-47 (_sampler: T = 0.8,
 * top-p 0.8), drawn on the device inside the captured step instead of on the
 * host after it. */
int tfa_top_p_sample_step(const float* logits, int64_t vocab, int64_t batch, const float* params,
                          const int64_t* seed, const int* inp, const int* prompt_len, int64_t* ids, int* pos,
                          int* sam, int64_t nsteps, int* err, hipStream_t stream);

/* ------------------------------------------ MLA decode, absorbed (MiniCPM3) */

/* Per sequence b (batch <= 65535): reduce the split-K partials part
 * [ks, batch, q_lora + 256 + 32] f32 of x_n . [W_q_a; W_kv_a]^T (each value
 * landing in bf16); q_n[b] = bf16(bf16(q_a * rsqrt(mean q_a^2 + eps)) * gamma_q_a);
 * latent_cache[b, pos[b]] = the same norm of kv_c with gamma_kv_a;
 * rope_cache[b, pos[b]] = rotate-half RoPE of the 32-wide rope slice at pos[b]
 * (bf16 products and sum). Caches are [batch, cap, 256] / [batch, cap, 32]
 * bf16; cos/sin [rope_rows, 32] bf16. A pos outside [0, cap) or the table sets
 * *err = 6 and skips the cache writes. q_lora <= 1024.
 * Replaces (absorbed form): examples/minicpm3_4b-cutedsl/model.py:220-250 (steps 1-4
 * of mla_attention), kernels/cute_gemv.py:246-286 (NORM_GEMV) and the kv half
 * of :291-347 (NORM_GEMV_PAIR). */
int tfa_mla_prep(const float* part, int64_t ks, int64_t batch, int64_t q_lora, const void* gamma_q_a,
                 const void* gamma_kv_a, float eps, const void* cos_t, const void* sin_t,
                 int64_t rope_rows, const int* pos, void* latent_cache, void* rope_cache, int64_t cap,
                 void* q_n, int* err, hipStream_t stream);

/* The absorbed query: from the split-K partials q_part [ks, batch, heads*96]
 * f32 of q_n . W_q_b^T (landing in bf16), q_abs[b, h, 0:256] =
 * bf16(W_UK_h^T q_nope) (f32 accumulate) and q_abs[b, h, 256:288] = RoPE of
 * q_rope at pos[b]. w_kv_b is [heads*128, 256] (out, in): rows h*128 .. +63
 * are W_UK_h, rows h*128+64 .. +127 are W_UV_h. batch <= 32, heads <= 48.
 * Replaces (absorbed form): the q half of kernels/cute_gemv.py:291-347 and the
 * q rotation of kernels/reference_ops.py:99-107. */
int tfa_mla_q_absorb(const float* q_part, int64_t ks, int64_t batch, int64_t heads, const void* w_kv_b,
                     const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos, void* q_abs,
                     int* err, hipStream_t stream);

/* The q_b projection and the absorbed query in one launch: q_up[b] =
 * bf16(q_n[b] . W_q_b^T) (f32 accumulate) for q_n [batch, q_lora] bf16 and
 * w_q_b [heads*96, q_lora] (out, in), then q_abs as tfa_mla_q_absorb writes it
 * from q_up. q_lora = 768, batch <= 32, heads <= 48; q_n, w_q_b and w_kv_b
 * 16-byte aligned. A position outside the rope table sets *err = 6 (row 0 used).
 * Replaces (absorbed form): examples/minicpm3_4b-cutedsl/model.py:232-236 (q_up =
 * q_n . w_q_b, split into nope | rope) with the q half of kernels/cute_gemv.py:291-347
 * and the q rotation of kernels/reference_ops.py:99-107. */
int tfa_mla_qb_absorb(const void* q_n, int64_t batch, int64_t heads, int64_t q_lora, const void* w_q_b,
                      const void* w_kv_b, const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos,
                      void* q_abs, int* err, hipStream_t stream);

/* One sequence's MLA prep, q_b projection and absorbed query in one launch:
 * from part = [q_a (768) | kv_c (256) | k_rope (32)] f32 (the single split-K
 * partial tfa_rmsnorm_gemv_f32 leaves), q_n = LoRA norm of q_a with gamma_q_a
 * (bit-equal to tfa_mla_prep's), latent_cache[pos[0]] and rope_cache[pos[0]]
 * written as tfa_mla_prep writes them (a pos outside [0, cap) or the rope table
 * sets *err = 6 and skips them), and q_abs [1, heads, 288] as tfa_mla_qb_absorb
 * computes it from q_n. q_lora = 768, heads <= 48; part, gamma_q_a, w_q_b and
 * w_kv_b 16-byte aligned.
 * Replaces: examples/minicpm3_4b-cutedsl/model.py:220-251 (steps 1-4 of
 * mla_attention at one sequence) with kernels/cute_gemv.py:246-347 (NORM_GEMV,
 * NORM_GEMV_PAIR) and the q rotation of kernels/reference_ops.py:99-107. */
int tfa_mla_prep_qb_absorb(const float* part, int64_t q_lora, const void* gamma_q_a, const void* gamma_kv_a,
                           float eps, const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos,
                           void* latent_cache, void* rope_cache, int64_t cap, const void* w_q_b, const void* w_kv_b,
                           int64_t heads, void* q_abs, int* err, hipStream_t stream);

/* Split attention of q_abs [batch, heads, 288] bf16 over slots 0..wr[b] of the
 * compressed cache on bf16 MFMA: s = scale * (q_abs . [latent | rope]) in f32,
 * per split (split positions: 32, 64, 96 or a multiple of 128 up to 1024) the softmax in
 * f32 with bf16 weights into the latent sum; op [batch, cap/split, heads, 256]
 * bf16 = the split's latent sum / its own weight sum, mp / lp [batch,
 * cap/split, heads] its max and sum. Only splits holding slots <= wr[b] are
 * written. A wr outside [0, cap) sets *err = 4 (clamped). q_abs, both caches and
 * op 16-byte aligned.
 * Replaces (absorbed form): kernels/cute_attention.py:56-200 (ROPE_ATTEND),
 * kernels/reference_ops.py:87-130 (rope_attend). */
int tfa_mla_attention(const void* q_abs, const void* latent_cache, const void* rope_cache, const int* wr,
                      int64_t batch, int64_t heads, int64_t cap, int64_t split, float scale, void* op,
                      float* mp, float* lp, int* err, hipStream_t stream);

/* Merge of tfa_mla_attention's splits per (head, sequence): weights
 * w_s = lp e^(mp - max), o_lat = sum_s w_s op_s / sum_s w_s (f32), then
 * attn[b, h*64 + v] = bf16(W_UV_h o_lat) over the splits holding slots <= wr[b].
 * op and w_kv_b 16-byte aligned.
 * Replaces (absorbed form): the 8-warp LSE merge of kernels/cute_attention.py:56-200
 * and the value half of W_kv_b applied per position in reference_ops.py:111-128. */
int tfa_mla_combine_up(const void* op, const float* mp, const float* lp, const int* wr, int64_t splits,
                       int64_t split, int64_t batch, int64_t heads, int64_t cap, const void* w_kv_b,
                       void* attn, hipStream_t stream);

/* Context splits (256 rows each) tfa_rope_attend uses for a cache of `cap` rows:
 * the row count of its op / mp / lp workspace. */
int64_t tfa_rope_attend_splits(int64_t cap);

/* MiniCPM3 decode attention over the assembled per-head cache (non-absorbed):
 * q_up [heads, nope + rope] and kv_up [heads, nope + v_dim] (this token's
 * [k_nope | v]) bf16, k_rope [rope] the unrotated shared key slice; cos / sin
 * [rope_rows, rope]; k_cache [cap, heads, nope + rope], v_cache [cap, heads,
 * v_dim] of which the first ctx[0] rows are context; scale bf16 [1].
 * q's rotary slice and k_rope are rotated at pos[0] (bf16 products and sum),
 * q is multiplied by scale in bf16, scores are f32 dots, the f32 softmax runs
 * over the context and the token itself, f32 weights into the value sum:
 * attn [heads * v_dim] bf16; k_new [heads, nope + rope] = [k_nope | rotated
 * k_rope] and v_new [heads, v_dim] (both optional). op / mp / lp: f32 workspace
 * [tfa_rope_attend_splits(cap), heads, v_dim] / [.., heads] (unused when cap = 0).
 * (nope + rope) % 8 == 0, <= 256; v_dim <= 128. err: 4 = ctx out of [0, cap],
 * 5 = pos out of [0, rope_rows).
 * Replaces examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:87-130
 * (rope_attend) and kernels/cute_attention.py:56-200 (ROPE_ATTEND). */
int tfa_rope_attend(const void* q_up, const void* kv_up, const void* k_rope, const void* cos_t,
                    const void* sin_t, int64_t rope_rows, const int* pos, const void* k_cache,
                    const void* v_cache, int64_t cap, const int* ctx, const void* scale,
                    int64_t heads, int64_t nope, int64_t rope, int64_t v_dim, float* op, float* mp,
                    float* lp, void* attn, void* k_new, void* v_new, int* err, hipStream_t stream);

/* tfa_rope_attend with no workspace argument: the same kernels, arguments and
 * results, with the split partials (op, then mp and lp) kept in a file-scope
 * device array of tfa_rope_attend_noalloc_max_floats() = 1,048,576 floats
 * (4 MiB) that each GPU the library runs on holds until the process ends.
 * Nothing is allocated, by the library or the caller.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 * Limit: tfa_rope_attend_splits(cap) * heads * (v_dim + 2) <= 1,048,576, else
 * TFA_ERR_CAPACITY (MiniCPM3's 40 heads x 64 value dims: cap <= 101,632).
 * The first call on a device resolves the array's address there
 * (hipGetSymbolAddress); make that call outside graph capture. Every call on
 * one GPU shares that GPU's array, so calls that overlap on one GPU (on two
 * streams, or from two threads) race; nothing in the array needs clearing,
 * since each call writes every partial it reads. */
int64_t tfa_rope_attend_noalloc_max_floats(void);
int tfa_rope_attend_noalloc(const void* q_up, const void* kv_up, const void* k_rope, const void* cos_t,
                            const void* sin_t, int64_t rope_rows, const int* pos, const void* k_cache,
                            const void* v_cache, int64_t cap, const int* ctx, const void* scale,
                            int64_t heads, int64_t nope, int64_t rope, int64_t v_dim, void* attn,
                            void* k_new, void* v_new, int* err, hipStream_t stream);

/* out[i, j] = bf16(residual[i, j] + bf16(bf16(sum_s part[s, i, j]) * alpha)) for
 * part [ks, m, n] f32 split-K partials (n % 8 == 0): the o_proj epilogue with
 * MiniCPM3's scale_depth residual.
 * Replaces: kernels/cute_gemv.py:430-495 (gemv_residual), reference_ops.py:63-65. */
int tfa_rows_residual(const float* part, int64_t ks, const void* residual, float alpha, void* out,
                      int64_t m, int64_t n, hipStream_t stream);

/* ------------------------------------------------- prefill (Qwen3.5 layer) */

/* Causal GQA attention over a whole prompt with the output gate:
 * out[n, h*256 + d] = bf16(bf16(o[n, h, d] / l) * bf16(sigmoid(gate[n, h, d]))),
 * o = sum_{j <= n} bf16(exp(s - m)) v[j, h / (heads/kv_heads)] over the f32
 * scores s = scale * q[n, h] . k[j, g] (bf16 MFMA, f32 accumulate). Element
 * (n, h, d) of q / gate sits at q + n*q_rs + h*q_hs + d (k, v likewise per kv
 * head), so q, gate, k and v can be read in place from the qkv projection's
 * output. head_dim 256; n a multiple of 128; q/k/v/gate/out strides multiples
 * of 8 (elements), every pointer 16-byte aligned.
 * Replaces: examples/qwen3_8_27b_prefill-tilelang/kernels/attention.py:313-438
 * (attention_ws / attention_tir), model.py:305-324 (Attention.attention). */
int tfa_prefill_attention(const void* q, int64_t q_rs, int64_t q_hs, const void* k, int64_t k_rs, int64_t k_hs,
                          const void* v, int64_t v_rs, int64_t v_hs, const void* gate, int64_t g_rs,
                          int64_t g_hs, void* out, int64_t o_rs, int64_t n, int64_t heads, int64_t kv_heads,
                          int64_t head_dim, float scale, hipStream_t stream);

/* C[m, n] = bf16(A[m, k] . B[n, k]^T) (residual == NULL) or
 * C = bf16(residual + bf16(A . B^T)) (residual [m, ldr]); bf16 in, f32 accumulate
 * on bf16 MFMA, the residual added in the kernel's epilogue. Row strides lda /
 * ldb / ldc in elements. m >= 1, n a multiple of 128, k of 64; lda, ldb
 * multiples of 8, ldc, ldr of 4; a, b 16-byte and c, residual 8-byte aligned.
 * Replaces: examples/qwen3_8_27b_prefill-tilelang/kernels/gemm.py:104-356 (gemm_kernel,
 * "residual" epilogue :193-198 -- model.py:326-333 Attention.o_proj). */
int tfa_gemm_nt(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                int64_t ldc, const void* residual, int64_t ldr, hipStream_t stream);

/* The qkv projection of the Qwen3.5 attention layer: out[n, (2*heads + 2*kv_heads)*256]
 * = hn[n, hidden] . w_qkv^T with w_qkv rows laid out [q_0 | gate_0 | ... | q_{H-1} |
 * gate_{H-1} | k_0..k_{G-1} | v_0..v_{G-1}] (256 rows each); then per token the q
 * and k slices get bf16(x * rsqrt(mean x^2 + eps) * (1 + gamma)) (f32) and
 * rotate-half RoPE on dims 0..rot-1 with cos/sin [n, rot] (bf16 products and
 * sum), all in the GEMM's epilogue. head_dim 256, rot 64; n >= 1, hidden a
 * multiple of 64.
 * Replaces: examples/qwen3_8_27b_prefill-tilelang/kernels/gemm.py:226-300 ("qk_norm_rope"
 * epilogue), model.py:271-303 (Attention.qkv), kernels/pack.py:48-64 (the layout). */
int tfa_qkv_norm_rope(const void* hn, const void* w_qkv, void* out, int64_t n, int64_t hidden, int64_t heads,
                      int64_t kv_heads, int64_t head_dim, const void* gamma_q, const void* gamma_k, float eps,
                      const void* cos_t, const void* sin_t, int64_t rot, hipStream_t stream);

/* ------------------------------------- prompt prefill (Qwen3-shaped decode model) */

/* C[m, n] = A[m, k] . B[n, k]^T in f32 (bf16 in, f32 accumulate, no rounding):
 * the prompt rows' projections, landed in bf16 by their consumers exactly as
 * the decode step lands its split-K partials (tfa_rows_norm, tfa_silu_mul and
 * tfa_prefill_qk_rope with ks = 1). The MFMA kernel of tfa_gemm_nt with an f32
 * store; m >= 1, n a multiple of 128, k of 64, lda / ldb multiples of 8.
 * Replaces: the per-token projection GEMVs of the prompt walk,
 * examples/qwen3_1_7b-tilelang/fast/engine.py:261-263 over fast/kernels.py:123-145
 * (gemv) -- the same products for every prompt row in one call. */
int tfa_gemm_nt_f32(const void* a, const void* b, float* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                    int64_t ldb, int64_t ldc, hipStream_t stream);

/* The same product with K split into ks equal ranges (ks in [1, 8], dividing k / 64):
 * range z lands, unrounded, in c + z * m * ldc, so c holds ks partials [ks, m, ldc]
 * whose consumers sum them in split order (tfa_rows_norm, tfa_swiglu_pairs_split
 * and tfa_prefill_qk_rope_split take ks). For few token rows, where the unsplit grid leaves
 * most CUs idle. Replaces the same products as tfa_gemm_nt_f32. */
int tfa_gemm_nt_f32_split(const void* a, const void* b, float* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                          int64_t ldb, int64_t ldc, int64_t ks, hipStream_t stream);

/* The split count tfa_gemm_nt_f32_split is fastest with for this shape (1 when
 * the unsplit grid fills the CUs). It is planned for MI355X's 256 CUs from the
 * shape alone, not from the device's reported CU count: the count fixes the
 * order the partials are summed in, so the same prompt prefills to the same
 * bits on any device. */
int64_t tfa_gemm_f32_splits(int64_t m, int64_t n, int64_t k);

/* SwiGLU of the prompt rows' fused gate|up product: gu f32 [rows, ld] with
 * column 2i = gate_i, 2i+1 = up_i (the interleaved decode weight layout);
 * act[r, i] = bf16(bf16(silu(bf16 g)) * bf16 u) -- the decode step's epilogue.
 * inter a multiple of 4; ld >= 2*inter, a multiple of 4; gu 16-byte aligned.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:547-572 (silu_mul) and the
 * SwiGLU prologue of :210-257 (gemv_silu), for every prompt row at once. */
int tfa_swiglu_pairs(const float* gu, int64_t ld, int64_t rows, int64_t inter, void* act, hipStream_t stream);

/* tfa_swiglu_pairs over ks f32 split-K partials gu [ks, rows, ld] (ks in [1, 8],
 * summed in split order before the landing), the output of
 * tfa_gemm_nt_f32_split. tfa_swiglu_pairs is this entry with ks = 1.
 * Replaces the same reference interfaces as tfa_swiglu_pairs. */
int tfa_swiglu_pairs_split(const float* gu, int64_t ks, int64_t ld, int64_t rows, int64_t inter, void* act,
                           hipStream_t stream);

/* Per-head norm + RoPE + cache write for the prompt rows of a batch: qkv f32
 * [batch * n, ldq] holds sequence b's row r at b * n + r (position pos0 + r),
 * columns [q (hq*128) | k (hkv*128) | v (hkv*128)]. Each head lands in bf16;
 * query heads get Qwen3RMSNorm(gamma_q) + rotate-half RoPE at the position and
 * go to q_out[(b*n + r), hq*128]; key heads the same with gamma_k into
 * k_cache[b, pos0 + r], value heads into v_cache[b, pos0 + r] (caches
 * [batch, cap, hkv*128]). The arithmetic of tfa_qk_rope_cache, so a prefilled
 * cache row is what the decode step would have written from the same
 * projection values. head_dim 128; pos0 + n <= cap and <= rope_rows.
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:328-411 (qk_rope_cache) run
 * once per prompt token by the walk (fast/engine.py:261-263). */
int tfa_prefill_qk_rope(const float* qkv, int64_t ldq, const void* gamma_q, const void* gamma_k, float eps_head,
                        const void* cos_t, const void* sin_t, int64_t rope_rows, int64_t batch, int64_t n,
                        int64_t pos0, void* k_cache, void* v_cache, int64_t cap, void* q_out, int64_t hq,
                        int64_t hkv, int64_t head_dim, hipStream_t stream);

/* tfa_prefill_qk_rope over ks f32 split-K partials qkv [ks, batch * n, ldq]
 * (ks in [1, 8], summed in split order before each head lands), the output of
 * tfa_gemm_nt_f32_split. tfa_prefill_qk_rope is this entry with ks = 1.
 * Replaces the same reference interface as tfa_prefill_qk_rope. */
int tfa_prefill_qk_rope_split(const float* qkv, int64_t ks, int64_t ldq, const void* gamma_q, const void* gamma_k,
                              float eps_head, const void* cos_t, const void* sin_t, int64_t rope_rows,
                              int64_t batch, int64_t n, int64_t pos0, void* k_cache, void* v_cache, int64_t cap,
                              void* q_out, int64_t hq, int64_t hkv, int64_t head_dim, hipStream_t stream);

/* Causal GQA attention of every row of a batch of prompts, no gate:
 * out[b, r, h*D + d] = bf16(o / l), o = sum_{j <= r} bf16(exp(s - m)) v[b, j, g],
 * s = scale * q[b, r, h] . k[b, j, g] (f32), g = h / (heads / kv_heads).
 * Element (b, r, h, d) of q sits at q + b*q_bs + r*q_rs + h*q_hs + d; k and v
 * likewise per kv head (the decode cache [batch, cap, kv_heads*D] is read in
 * place: k_rs = kv_heads*D, k_hs = D, k_bs = cap*kv_heads*D); out rows at
 * out + b*o_bs + r*o_rs. head_dim 128 or 256; any n >= 1; q/k/v/out strides
 * multiples of 8 (elements), every pointer 16-byte aligned.
 * Replaces: the per-token attention of the prompt walk,
 * examples/qwen3_1_7b-tilelang/fast/kernels.py:418-540 (attn_partial + merge) at each
 * position 0..n-1 (fast/engine.py:261-263); ref_src/model.py:171-215 (self_attention). */
int tfa_causal_attention(const void* q, int64_t q_rs, int64_t q_hs, int64_t q_bs, const void* k, int64_t k_rs,
                         int64_t k_hs, int64_t k_bs, const void* v, int64_t v_rs, int64_t v_hs, int64_t v_bs,
                         void* out, int64_t o_rs, int64_t o_bs, int64_t batch, int64_t n, int64_t heads,
                         int64_t kv_heads, int64_t head_dim, float scale, hipStream_t stream);

/* ------------------------------------------------------------ measurement */

/* dst[0:bytes) = src[0:bytes) with the decode kernels' own access pattern
 * (16-byte non-temporal loads, 16-byte stores, 64 KiB per block). Used to
 * re-measure the sustained HBM bandwidth and as the calibration dispatch for
 * hardware byte counters. No counterpart in the reference (its READMEs quote
 * H200 nominal bandwidth). bytes % 16 == 0. */
int tfa_copy_stream(const void* src, void* dst, int64_t bytes, hipStream_t stream);

/* Measurement utility: the decode GEMV's weight stream alone over w [rows, k]
 * bf16 -- one-shot 256-thread blocks of rows_per_block (2, 4, 6 or 8) rows,
 * each wave a contiguous quarter of every row in 16-byte non-temporal loads --
 * folded to one value per block in out [ceil(rows / rows_per_block)] f32 (its
 * value means nothing). Its time per launch is the floor of the GEMV's access
 * pattern on a matrix of that shape. No counterpart in the reference (a
 * measurement of this device). */
int tfa_read_rows(const void* w, int64_t rows, int64_t k, int64_t rows_per_block, float* out, hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* TILEFOUNDRY_AMD_H_ */
