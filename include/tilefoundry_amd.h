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

/* Greedy pick + sample step on the device: best = argmax over the block
 * winners (lowest index on ties); sam[pos] = best; ids[0] = pos+1 < prompt_len ?
 * inp[pos+1] : best; pos += 1. inp / sam are int32 [nsteps].
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:591-637 (sample_step). */
int tfa_sample_step(const float* block_val, const int* block_idx, int64_t nblocks, const int* inp,
                    const int* prompt_len, int64_t* ids, int* pos, int* sam, int64_t nsteps,
                    int* err, hipStream_t stream);

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

/* Split-KV GQA decode attention (head_dim 128), caches [cap, hkv*128]
 * position-major, attending slots 0..wr[0]. Scores scaled by `scale` in f32
 * after the dot; softmax in f32 per split of `split` (64, 128 or 256) slots;
 * bf16 weights into P.V. Partials op [cap/split, hq, 128], mp / lp
 * [cap/split, hq]; splits past wr are left untouched unless `neutral`
 * (then m = -1e30, l = 0, o = 0).
 * Prepared mode (gamma_q == NULL): q is the final query [hq*128] and the cache
 * already holds slot wr. Fused mode: q is the raw [q | k] projection
 * [(hq+hkv)*128]; each query head gets Qwen3RMSNorm (gamma_q, eps_head) and
 * rotate-half RoPE at pos[0] (cos / sin [rope_rows, 128]); the new key gets the
 * same with gamma_k and is written to k_cache row wr[0].
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501 (attn_partial)
 * and :328-411 (qk_rope_cache). */
int tfa_decode_attention(const void* q, const void* gamma_q, const void* gamma_k, float eps_head,
                         const void* cos_t, const void* sin_t, int64_t rope_rows, void* k_cache,
                         const void* v_cache, const int* pos, const int* wr, int64_t hq,
                         int64_t hkv, int64_t head_dim, int64_t cap, int64_t split, float scale,
                         float* op, float* mp, float* lp, int neutral, int* err,
                         hipStream_t stream);

/* out[h*D + d] = bf16(sum_s op[s,h,d] e^(mp[s,h]-M) / sum_s lp[s,h] e^(mp[s,h]-M))
 * over all `splits`, or (wr != NULL) over the splits holding slots 0..wr[0].
 * Replaces: examples/qwen3_1_7b-tilelang/fast/kernels.py:504-540 (attn_combine). */
int tfa_attn_combine(const float* op, const float* mp, const float* lp, void* out, int64_t splits,
                     int64_t hq, int64_t head_dim, const int* wr, int64_t split,
                     hipStream_t stream);

/* ------------------------------------------------------------ measurement */

/* dst[0:bytes) = src[0:bytes) with the decode kernels' own access pattern
 * (16-byte non-temporal loads, 16-byte stores, 64 KiB per block). Used to
 * re-measure the sustained HBM bandwidth and as the calibration dispatch for
 * hardware byte counters. No counterpart in the reference (its READMEs quote
 * H200 nominal bandwidth). bytes % 16 == 0. */
int tfa_copy_stream(const void* src, void* dst, int64_t bytes, hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* TILEFOUNDRY_AMD_H_ */
