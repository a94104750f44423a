// Thin PyTorch-ROCm extension over the C ABI in include/tilefoundry_amd.h.
//
// Each binding checks what the C ABI cannot see -- device, dtype, contiguity
// and that every tensor's size agrees with the dimensions passed down -- then
// calls the entry point on torch's current HIP stream. A status other than
// TFA_OK becomes ValueError (bad arguments) or RuntimeError (a refused launch),
// carrying the entry point's own message.
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <sstream>
#include <string>

#include "tilefoundry_amd.h"

namespace {

using at::Tensor;

hipStream_t stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void raise_status(int st) {
  if (st == TFA_OK) return;
  std::string msg = tfa_last_error();
  if (msg.empty()) msg = tfa_status_string(st);
  if (st == TFA_ERR_LAUNCH) throw std::runtime_error(msg);
  throw pybind11::value_error(msg);
}

[[noreturn]] void bad(const std::string& m) { throw pybind11::value_error(m); }

void need(const Tensor& t, const char* name, at::ScalarType dt, int64_t numel = -1) {
  if (!t.defined()) bad(std::string(name) + ": tensor required");
  if (!t.is_cuda()) bad(std::string(name) + ": must be a GPU tensor");
  if (t.scalar_type() != dt) {
    std::ostringstream o;
    o << name << ": dtype " << t.scalar_type() << ", expected " << dt;
    bad(o.str());
  }
  if (!t.is_contiguous()) bad(std::string(name) + ": must be contiguous");
  if (numel >= 0 && t.numel() != numel) {
    std::ostringstream o;
    o << name << ": has " << t.numel() << " elements, expected " << numel;
    bad(o.str());
  }
}

const auto BF = at::kBFloat16;
const auto F32 = at::kFloat;
const auto I32 = at::kInt;
const auto I64 = at::kLong;

// ------------------------------------------------------------------ norms
int64_t last_dim(const Tensor& t) { return t.dim() == 0 ? 1 : t.size(-1); }

void rms_norm(const Tensor& x, const Tensor& gamma, const Tensor& y, double eps, int64_t mode) {
  const int64_t H = last_dim(x);
  const int64_t rows = H ? x.numel() / H : 0;
  need(x, "x", BF);
  need(gamma, "gamma", BF, H);
  need(y, "y", BF, x.numel());
  raise_status(tfa_rms_norm(x.data_ptr(), gamma.data_ptr(), y.data_ptr(), rows, H, (float)eps,
                            (int)mode, stream_of(x)));
}

void rms_norm_div(const Tensor& x, const Tensor& gamma, const Tensor& y, double eps, double divisor) {
  const int64_t H = last_dim(x);
  const int64_t rows = H ? x.numel() / H : 0;
  need(x, "x", BF);
  need(gamma, "gamma", BF, H);
  need(y, "y", BF, x.numel());
  raise_status(tfa_rms_norm_div(x.data_ptr(), gamma.data_ptr(), y.data_ptr(), rows, H, (float)eps,
                                (float)divisor, stream_of(x)));
}

void add_rms_norm(const Tensor& x, const Tensor& residual, const Tensor& gamma, const Tensor& y,
                  const Tensor& residual_out, double eps, int64_t mode) {
  const int64_t H = last_dim(x);
  const int64_t rows = H ? x.numel() / H : 0;
  need(x, "x", BF);
  need(residual, "residual", BF, x.numel());
  need(gamma, "gamma", BF, H);
  need(y, "y", BF, x.numel());
  need(residual_out, "residual_out", BF, x.numel());
  raise_status(tfa_add_rms_norm(x.data_ptr(), residual.data_ptr(), gamma.data_ptr(), y.data_ptr(),
                                residual_out.data_ptr(), rows, H, (float)eps, (int)mode,
                                stream_of(x)));
}

void resid_rms_norm_partials(const Tensor& a, const Tensor& partials, const Tensor& gamma,
                             const Tensor& h_out, const Tensor& xn, double eps) {
  const int64_t H = a.numel();
  need(a, "A", BF);
  need(partials, "P", F32);
  if (partials.dim() != 2 || partials.size(1) != H) bad("P: expected shape (SK, H)");
  need(gamma, "G", BF, H);
  need(h_out, "Hout", BF, H);
  need(xn, "Xn", BF, H);
  raise_status(tfa_resid_rms_norm_partials(a.data_ptr(), partials.data_ptr<float>(),
                                           partials.size(0), gamma.data_ptr(), h_out.data_ptr(),
                                           xn.data_ptr(), H, (float)eps, stream_of(a)));
}

// -------------------------------------------------------------- decode
using OptT = std::optional<Tensor>;

const void* opt_ptr(const OptT& t) { return (t && t->defined()) ? t->data_ptr() : nullptr; }
template <typename T>
T* opt_ptr_t(const OptT& t) { return (t && t->defined()) ? static_cast<T*>(t->data_ptr()) : nullptr; }

void need_mat(const Tensor& w, const char* name, int64_t n, int64_t k) {
  need(w, name, BF);
  if (w.dim() != 2 || w.size(0) != n || w.size(1) != k) {
    std::ostringstream o;
    o << name << ": expected shape (" << n << ", " << k << "), got " << w.sizes();
    bad(o.str());
  }
}

void gemv(const Tensor& x, const Tensor& w, const Tensor& y) {
  need(x, "x", BF);
  const int64_t K = x.numel();
  if (w.dim() != 2) bad("w: expected a 2-D (N, K) weight");
  const int64_t N = w.size(0);
  need_mat(w, "w", N, K);
  const bool f32 = y.scalar_type() == F32;
  need(y, "y", f32 ? F32 : BF, N);
  raise_status(tfa_gemv(x.data_ptr(), w.data_ptr(), y.data_ptr(), N, K, f32 ? 1 : 0, stream_of(x)));
}

void rmsnorm_gemv(const Tensor& h, const Tensor& gamma, double eps, const Tensor& w, const Tensor& y) {
  need(h, "h", BF);
  const int64_t K = h.numel();
  need(gamma, "gamma", BF, K);
  if (w.dim() != 2) bad("w: expected a 2-D (N, K) weight");
  const int64_t N = w.size(0);
  need_mat(w, "w", N, K);
  need(y, "y", BF, N);
  raise_status(tfa_rmsnorm_gemv(h.data_ptr(), gamma.data_ptr(), (float)eps, w.data_ptr(),
                                y.data_ptr(), N, K, stream_of(h)));
}

void rmsnorm_gemv_f32(const Tensor& h, const Tensor& gamma, double eps, const Tensor& w, const Tensor& y) {
  need(h, "h", BF);
  const int64_t K = h.numel();
  need(gamma, "gamma", BF, K);
  if (w.dim() != 2) bad("w: expected a 2-D (N, K) weight");
  const int64_t N = w.size(0);
  need_mat(w, "w", N, K);
  need(y, "y", F32, N);
  raise_status(tfa_rmsnorm_gemv_f32(h.data_ptr(), gamma.data_ptr(), (float)eps, w.data_ptr(),
                                    y.data_ptr<float>(), N, K, stream_of(h)));
}

// One sequence: part [q_lora + 288] f32, latent (1, cap, 256), rope (1, cap, 32),
// w_q_b [N, q_lora], q_part [N] f32.
void mla_prep_q_gemv(const Tensor& part, const Tensor& gamma_q_a, const Tensor& gamma_kv_a, double eps,
                     const Tensor& cos, const Tensor& sin, const Tensor& pos, const Tensor& latent,
                     const Tensor& rope, const Tensor& w_q_b, const Tensor& q_part, const OptT& err) {
  need(pos, "pos", I32, 1);
  need(latent, "latent", BF);
  if (latent.dim() != 3 || latent.size(0) != 1 || latent.size(2) != 256) bad("latent: expected (1, cap, 256)");
  const int64_t cap = latent.size(1);
  need(rope, "rope", BF, cap * 32);
  need(gamma_kv_a, "gamma_kv_a", BF, 256);
  need(gamma_q_a, "gamma_q_a", BF);
  const int64_t QA = gamma_q_a.numel();
  need(part, "part", F32, QA + 288);
  if (w_q_b.dim() != 2) bad("w_q_b: expected a 2-D (N, q_lora) weight");
  const int64_t N = w_q_b.size(0);
  need_mat(w_q_b, "w_q_b", N, QA);
  need(q_part, "q_part", F32, N);
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (cos.numel() % 32 != 0) bad("cos: expected (rows, 32)");
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_mla_prep_q_gemv(part.data_ptr<float>(), QA, gamma_q_a.data_ptr(), gamma_kv_a.data_ptr(),
                                   (float)eps, cos.data_ptr(), sin.data_ptr(), cos.numel() / 32,
                                   pos.data_ptr<int>(), latent.data_ptr(), rope.data_ptr(), cap,
                                   w_q_b.data_ptr(), q_part.data_ptr<float>(), N, opt_ptr_t<int>(err),
                                   stream_of(pos)));
}

void gemv_residual(const Tensor& x, const Tensor& w, const Tensor& residual, const OptT& alpha,
                   const Tensor& y) {
  need(x, "x", BF);
  const int64_t K = x.numel();
  if (w.dim() != 2) bad("w: expected a 2-D (N, K) weight");
  const int64_t N = w.size(0);
  need_mat(w, "w", N, K);
  need(residual, "residual", BF, N);
  need(y, "y", BF, N);
  if (alpha) need(*alpha, "alpha", BF, 1);
  if (y.data_ptr() == residual.data_ptr()) bad("y must not alias residual");
  raise_status(tfa_gemv_residual(x.data_ptr(), w.data_ptr(), residual.data_ptr(), opt_ptr(alpha),
                                 y.data_ptr(), N, K, stream_of(x)));
}

void rmsnorm_gemv_swiglu(const Tensor& h, const Tensor& gamma, double eps, const Tensor& w_gu,
                         const Tensor& act) {
  need(h, "h", BF);
  const int64_t K = h.numel();
  need(gamma, "gamma", BF, K);
  const int64_t I = act.numel();
  need_mat(w_gu, "w_gu", 2 * I, K);
  need(act, "act", BF, I);
  raise_status(tfa_rmsnorm_gemv_swiglu(h.data_ptr(), gamma.data_ptr(), (float)eps, w_gu.data_ptr(),
                                       act.data_ptr(), I, K, stream_of(h)));
}

void lm_head_argmax(const Tensor& h, const OptT& gamma, double eps, const Tensor& w,
                    const Tensor& logits, const Tensor& block_val, const Tensor& block_idx) {
  need(h, "h", BF);
  const int64_t K = h.numel();
  if (gamma) need(*gamma, "gamma", BF, K);
  if (w.dim() != 2) bad("w: expected a 2-D (V, K) weight");
  const int64_t V = w.size(0);
  need_mat(w, "w", V, K);
  need(logits, "logits", F32, V);
  const int64_t nb = tfa_lm_head_blocks(V);
  need(block_val, "block_val", F32, nb);
  need(block_idx, "block_idx", I32, nb);
  raise_status(tfa_lm_head_argmax(h.data_ptr(), opt_ptr(gamma), (float)eps, w.data_ptr(), V, K,
                                  logits.data_ptr<float>(), block_val.data_ptr<float>(),
                                  block_idx.data_ptr<int>(), stream_of(h)));
}

void sample_step(const Tensor& block_val, const Tensor& block_idx, const Tensor& inp,
                 const Tensor& prompt_len, const Tensor& ids, const Tensor& pos, const Tensor& sam,
                 const OptT& err) {
  need(block_val, "block_val", F32);
  need(block_idx, "block_idx", I32, block_val.numel());
  need(inp, "inp", I32);
  need(sam, "sam", I32, inp.numel());
  need(prompt_len, "prompt_len", I32, 1);
  need(ids, "ids", I64, 1);
  need(pos, "pos", I32, 1);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_sample_step(block_val.data_ptr<float>(), block_idx.data_ptr<int>(),
                               block_val.numel(), inp.data_ptr<int>(), prompt_len.data_ptr<int>(),
                               ids.data_ptr<int64_t>(), pos.data_ptr<int>(), sam.data_ptr<int>(),
                               inp.numel(), opt_ptr_t<int>(err), stream_of(block_val)));
}

void decode_qkv(const OptT& h, const OptT& table, const OptT& ids, const OptT& h_copy,
                const Tensor& gamma_in, double eps, const Tensor& w_qkv, int64_t n_qk,
                const Tensor& qk_out, const Tensor& wr, const Tensor& v_cache, const OptT& err) {
  const int64_t H = gamma_in.numel();
  need(gamma_in, "gamma_in", BF, H);
  int64_t vocab = 0;
  if (table) {
    need(*table, "table", BF);
    if (table->dim() != 2 || table->size(1) != H) bad("table: expected (V, hidden)");
    vocab = table->size(0);
    if (!ids || !h_copy) bad("embed mode needs ids and h_copy");
    need(*ids, "ids", I64, 1);
    need(*h_copy, "h_copy", BF, H);
  } else {
    if (!h) bad("h required when no table is given");
    need(*h, "h", BF, H);
  }
  if (w_qkv.dim() != 2) bad("w_qkv: expected (n_qk + n_v, hidden)");
  const int64_t n_v = w_qkv.size(0) - n_qk;
  if (n_v <= 0) bad("w_qkv has no value rows");
  need_mat(w_qkv, "w_qkv", n_qk + n_v, H);
  need(qk_out, "qk_out", BF, n_qk);
  need(wr, "wr", I32, 1);
  need(v_cache, "v_cache", BF);
  if (v_cache.numel() % n_v != 0) bad("v_cache: size is not a multiple of the value row");
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_decode_qkv(opt_ptr(h), opt_ptr(table), opt_ptr_t<const int64_t>(ids), vocab,
                              opt_ptr_t<void>(h_copy), gamma_in.data_ptr(), (float)eps,
                              w_qkv.data_ptr(), H, n_qk, n_v, qk_out.data_ptr(), wr.data_ptr<int>(),
                              v_cache.data_ptr(), v_cache.numel() / n_v, opt_ptr_t<int>(err),
                              stream_of(gamma_in)));
}

void decode_attention(const OptT& q, const OptT& qkv_part, const OptT& gamma_q,
                      const OptT& gamma_k, double eps_head, const OptT& cos_t, const OptT& sin_t,
                      const Tensor& k_cache, const Tensor& v_cache, const OptT& pos,
                      const Tensor& wr, int64_t hq, int64_t hkv, int64_t split, double scale,
                      const Tensor& op, const Tensor& mp, const Tensor& lp, bool neutral,
                      const OptT& err) {
  const int64_t D = 128;
  const bool fused = gamma_q.has_value();
  need(wr, "wr", I32);
  const int64_t B = wr.numel();
  int64_t ks = 0;
  if (qkv_part) {
    if (!fused) bad("qkv_part needs the fused-mode operands");
    need(*qkv_part, "qkv_part", F32);
    const int64_t per = B * (hq + 2 * hkv) * D;
    if (qkv_part->numel() % per != 0) bad("qkv_part: expected (ks, batch, (hq+2hkv)*128)");
    ks = qkv_part->numel() / per;
  } else {
    if (!q) bad("q required");
    need(*q, "q", BF, B * (fused ? hq + hkv : hq) * D);
  }
  int64_t rope_rows = 0;
  if (fused) {
    if (!gamma_k || !cos_t || !sin_t || !pos) bad("fused mode needs gamma_k, cos, sin and pos");
    need(*gamma_q, "gamma_q", BF, D);
    need(*gamma_k, "gamma_k", BF, D);
    need(*cos_t, "cos", BF);
    need(*sin_t, "sin", BF, cos_t->numel());
    if (cos_t->dim() != 2 || cos_t->size(1) != D) bad("cos: expected (rows, 128)");
    rope_rows = cos_t->size(0);
    need(*pos, "pos", I32, B);
  }
  need(k_cache, "k_cache", BF);
  need(v_cache, "v_cache", BF, k_cache.numel());
  if (k_cache.numel() % (B * hkv * D) != 0) bad("k_cache: size is not a multiple of batch*hkv*128");
  const int64_t cap = k_cache.numel() / (B * hkv * D);
  if (split <= 0 || cap % split != 0) bad("cache capacity must be a multiple of the split");
  const int64_t ns = cap / split;
  need(op, "op", F32, B * ns * hq * D);
  need(mp, "mp", F32, B * ns * hq);
  need(lp, "lp", F32, B * ns * hq);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_decode_attention(
      opt_ptr(q), opt_ptr_t<const float>(qkv_part), ks, opt_ptr(gamma_q), opt_ptr(gamma_k),
      (float)eps_head, opt_ptr(cos_t), opt_ptr(sin_t), rope_rows, k_cache.data_ptr(),
      v_cache.data_ptr(), opt_ptr_t<const int>(pos), wr.data_ptr<int>(), B, hq, hkv, D, cap, split,
      (float)scale, op.data_ptr<float>(), mp.data_ptr<float>(), lp.data_ptr<float>(),
      neutral ? 1 : 0, opt_ptr_t<int>(err), stream_of(k_cache)));
}

void attn_combine(const Tensor& op, const Tensor& mp, const Tensor& lp, const Tensor& out,
                  const OptT& wr, int64_t split) {
  need(mp, "Mp", F32);
  if (mp.dim() != 2 && mp.dim() != 3) bad("Mp: expected ([batch,] NS, HQ)");
  const int64_t B = mp.dim() == 3 ? mp.size(0) : 1;
  const int64_t ns = mp.size(-2), hq = mp.size(-1);
  need(lp, "Lp", F32, B * ns * hq);
  need(op, "Op", F32);
  if (op.numel() % (B * ns * hq) != 0) bad("Op: expected ([batch,] NS, HQ, D)");
  const int64_t D = op.numel() / (B * ns * hq);
  need(out, "O", BF, B * hq * D);
  if (wr) need(*wr, "wr", I32, B);
  raise_status(tfa_attn_combine(op.data_ptr<float>(), mp.data_ptr<float>(), lp.data_ptr<float>(),
                                out.data_ptr(), ns, B, hq, D, opt_ptr_t<const int>(wr), split,
                                stream_of(op)));
}

// ---------------------------------------------------------- batched decode
void skinny_gemm(const Tensor& x, const Tensor& w, int64_t ks, int64_t epilogue, const OptT& part,
                 const OptT& act, const OptT& logits, const OptT& block_val,
                 const OptT& block_idx) {
  need(x, "x", BF);
  if (x.dim() != 2) bad("x: expected (m, k)");
  const int64_t M = x.size(0), K = x.size(1);
  if (w.dim() != 2) bad("w: expected (n, k)");
  const int64_t N = w.size(0);
  need_mat(w, "w", N, K);
  if (epilogue == 0) {
    if (!part) bad("partial epilogue needs part");
    need(*part, "part", F32, ks * M * N);
  } else if (epilogue == 1) {
    if (!act) bad("swiglu epilogue needs act");
    need(*act, "act", BF, M * (N / 2));
  } else if (epilogue == 2 || epilogue == 3) {
    if (!block_val || !block_idx) bad("argmax epilogue needs block_val, block_idx");
    if (logits) need(*logits, "logits", F32, M * N);
    const int64_t nb = tfa_skinny_blocks(N);
    need(*block_val, "block_val", F32, M * nb);
    need(*block_idx, "block_idx", I32, M * nb);
  }
  raise_status(tfa_skinny_gemm(x.data_ptr(), w.data_ptr(), M, N, K, ks, (int)epilogue,
                               opt_ptr_t<float>(part), opt_ptr_t<void>(act), opt_ptr_t<float>(logits),
                               opt_ptr_t<float>(block_val), opt_ptr_t<int>(block_idx),
                               stream_of(x)));
}

void rows_norm(const OptT& table, const OptT& ids, const OptT& h_in, const OptT& part,
               const Tensor& h_out, const Tensor& gamma, const Tensor& xn, double eps,
               const OptT& err) {
  need(h_out, "h_out", BF);
  if (h_out.dim() != 2) bad("h_out: expected (m, hidden)");
  const int64_t M = h_out.size(0), H = h_out.size(1);
  need(gamma, "gamma", BF, H);
  need(xn, "xn", BF, M * H);
  int64_t vocab = 0, ks = 0;
  if (table) {
    need(*table, "table", BF);
    if (table->dim() != 2 || table->size(1) != H) bad("table: expected (V, hidden)");
    vocab = table->size(0);
    if (!ids) bad("embed mode needs ids");
    need(*ids, "ids", I64, M);
  } else {
    if (!h_in || !part) bad("residual mode needs h_in and part");
    need(*h_in, "h_in", BF, M * H);
    need(*part, "part", F32);
    if (part->numel() % (M * H) != 0) bad("part: expected (ks, m, hidden)");
    ks = part->numel() / (M * H);
  }
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_rows_norm(opt_ptr(table), opt_ptr_t<const int64_t>(ids), vocab, opt_ptr(h_in),
                             opt_ptr_t<const float>(part), ks, h_out.data_ptr(), gamma.data_ptr(),
                             xn.data_ptr(), M, H, (float)eps, opt_ptr_t<int>(err), stream_of(h_out)));
}

void batch_sample_step(const Tensor& block_val, const Tensor& block_idx, const Tensor& inp,
                       const Tensor& prompt_len, const Tensor& ids, const Tensor& pos,
                       const Tensor& sam, const OptT& err) {
  need(pos, "pos", I32);
  const int64_t B = pos.numel();
  need(block_val, "block_val", F32);
  if (block_val.numel() % B != 0) bad("block_val: expected (batch, nblocks)");
  const int64_t nb = block_val.numel() / B;
  need(block_idx, "block_idx", I32, B * nb);
  need(inp, "inp", I32);
  if (inp.numel() % B != 0) bad("inp: expected (batch, nsteps)");
  const int64_t nsteps = inp.numel() / B;
  need(sam, "sam", I32, B * nsteps);
  need(prompt_len, "prompt_len", I32, B);
  need(ids, "ids", I64, B);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_batch_sample_step(block_val.data_ptr<float>(), block_idx.data_ptr<int>(), nb, B,
                                     inp.data_ptr<int>(), prompt_len.data_ptr<int>(),
                                     ids.data_ptr<int64_t>(), pos.data_ptr<int>(), sam.data_ptr<int>(),
                                     nsteps, opt_ptr_t<int>(err), stream_of(pos)));
}

void skinny_gemm_residual(const Tensor& x, const Tensor& w, const Tensor& res, const Tensor& h_out,
                          const Tensor& ssq) {
  need(x, "x", BF);
  need(w, "w", BF);
  if (x.dim() != 2 || w.dim() != 2 || x.size(1) != w.size(1)) bad("skinny_gemm_residual: x [m, k], w [n, k]");
  const int64_t m = x.size(0), n = w.size(0), k = w.size(1);
  need(res, "res", BF, m * n);
  need(h_out, "h_out", BF, m * n);
  need(ssq, "ssq", F32, tfa_skinny_residual_blocks(n) * m);
  raise_status(tfa_skinny_gemm_residual(x.data_ptr(), w.data_ptr(), m, n, k, res.data_ptr(), h_out.data_ptr(),
                                        ssq.data_ptr<float>(), stream_of(x)));
}

void skinny_gemm_norm_swiglu(const Tensor& h, const Tensor& w, const Tensor& ssq, const Tensor& gamma, double eps,
                             const Tensor& act) {
  need(h, "h", BF);
  need(w, "w", BF);
  if (h.dim() != 2 || w.dim() != 2 || h.size(1) != w.size(1)) bad("skinny_gemm_norm_swiglu: h [m, k], w [n, k]");
  const int64_t m = h.size(0), n = w.size(0), k = w.size(1);
  need(ssq, "ssq", F32);
  if (ssq.numel() % m != 0) bad("ssq: expected (blocks, m)");
  need(gamma, "gamma", BF, k);
  need(act, "act", BF, m * (n / 2));
  raise_status(tfa_skinny_gemm_norm_swiglu(h.data_ptr(), w.data_ptr(), m, n, k, ssq.data_ptr<float>(),
                                           ssq.numel() / m, gamma.data_ptr(), (float)eps, act.data_ptr(),
                                           stream_of(h)));
}

void top_p_sample_step(const Tensor& logits, const Tensor& params, const Tensor& seed, const Tensor& inp,
                       const Tensor& prompt_len, const Tensor& ids, const Tensor& pos, const Tensor& sam,
                       const OptT& err) {
  need(pos, "pos", I32);
  const int64_t B = pos.numel();
  need(logits, "logits", F32);
  if (logits.numel() % B != 0) bad("logits: expected (batch, vocab)");
  const int64_t V = logits.numel() / B;
  need(params, "params", F32, 2);
  need(seed, "seed", I64, 1);
  need(inp, "inp", I32);
  if (inp.numel() % B != 0) bad("inp: expected (batch, nsteps)");
  const int64_t nsteps = inp.numel() / B;
  need(sam, "sam", I32, B * nsteps);
  need(prompt_len, "prompt_len", I32, B);
  need(ids, "ids", I64, B);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_top_p_sample_step(logits.data_ptr<float>(), V, B, params.data_ptr<float>(),
                                     seed.data_ptr<int64_t>(), inp.data_ptr<int>(), prompt_len.data_ptr<int>(),
                                     ids.data_ptr<int64_t>(), pos.data_ptr<int>(), sam.data_ptr<int>(), nsteps,
                                     opt_ptr_t<int>(err), stream_of(pos)));
}

// ------------------------------------------------------------------ MLA
// part [ks, B, q_lora + 288] f32; latent [B, cap, 256], rope [B, cap, 32] bf16.
void mla_prep(const Tensor& part, const Tensor& gamma_q_a, const Tensor& gamma_kv_a, double eps,
              const Tensor& cos, const Tensor& sin, const Tensor& pos, const Tensor& latent,
              const Tensor& rope, const Tensor& q_n, const OptT& err) {
  need(pos, "pos", I32);
  const int64_t B = pos.numel();
  need(latent, "latent", BF);
  need(rope, "rope", BF);
  if (latent.dim() != 3 || latent.size(0) != B || latent.size(2) != 256) bad("latent: expected (batch, cap, 256)");
  const int64_t cap = latent.size(1);
  need(rope, "rope", BF, B * cap * 32);
  need(gamma_kv_a, "gamma_kv_a", BF, 256);
  need(gamma_q_a, "gamma_q_a", BF);
  const int64_t QA = gamma_q_a.numel();
  need(q_n, "q_n", BF, B * QA);
  need(part, "part", F32);
  if (part.numel() % (B * (QA + 288)) != 0) bad("part: expected (ks, batch, q_lora + 288)");
  const int64_t ks = part.numel() / (B * (QA + 288));
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (cos.numel() % 32 != 0) bad("cos: expected (rows, 32)");
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_mla_prep(part.data_ptr<float>(), ks, B, QA, gamma_q_a.data_ptr(), gamma_kv_a.data_ptr(),
                            (float)eps, cos.data_ptr(), sin.data_ptr(), cos.numel() / 32, pos.data_ptr<int>(),
                            latent.data_ptr(), rope.data_ptr(), cap, q_n.data_ptr(), opt_ptr_t<int>(err),
                            stream_of(pos)));
}

// q_part [ks, B, H*96] f32, w_kv_b [H*128, 256], q_abs [B, H, 288] bf16.
void mla_q_absorb(const Tensor& q_part, const Tensor& w_kv_b, const Tensor& cos, const Tensor& sin,
                  const Tensor& pos, const Tensor& q_abs, const OptT& err) {
  need(pos, "pos", I32);
  const int64_t B = pos.numel();
  need(q_abs, "q_abs", BF);
  if (q_abs.dim() != 3 || q_abs.size(0) != B || q_abs.size(2) != 288) bad("q_abs: expected (batch, heads, 288)");
  const int64_t H = q_abs.size(1);
  need_mat(w_kv_b, "w_kv_b", H * 128, 256);
  need(q_part, "q_part", F32);
  if (q_part.numel() % (B * H * 96) != 0) bad("q_part: expected (ks, batch, heads*96)");
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_mla_q_absorb(q_part.data_ptr<float>(), q_part.numel() / (B * H * 96), B, H,
                                w_kv_b.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.numel() / 32,
                                pos.data_ptr<int>(), q_abs.data_ptr(), opt_ptr_t<int>(err), stream_of(pos)));
}

// q_n [B, 768] bf16, w_q_b [H*96, 768], w_kv_b [H*128, 256], q_abs [B, H, 288] bf16.
void mla_qb_absorb(const Tensor& q_n, const Tensor& w_q_b, const Tensor& w_kv_b, const Tensor& cos,
                   const Tensor& sin, const Tensor& pos, const Tensor& q_abs, const OptT& err) {
  need(pos, "pos", I32);
  const int64_t B = pos.numel();
  need(q_abs, "q_abs", BF);
  if (q_abs.dim() != 3 || q_abs.size(0) != B || q_abs.size(2) != 288) bad("q_abs: expected (batch, heads, 288)");
  const int64_t H = q_abs.size(1);
  need(q_n, "q_n", BF);
  if (q_n.dim() != 2 || q_n.size(0) != B) bad("q_n: expected (batch, q_lora)");
  const int64_t QL = q_n.size(1);
  need_mat(w_q_b, "w_q_b", H * 96, QL);
  need_mat(w_kv_b, "w_kv_b", H * 128, 256);
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (cos.numel() % 32 != 0) bad("cos: expected (rows, 32)");
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_mla_qb_absorb(q_n.data_ptr(), B, H, QL, w_q_b.data_ptr(), w_kv_b.data_ptr(), cos.data_ptr(),
                                 sin.data_ptr(), cos.numel() / 32, pos.data_ptr<int>(), q_abs.data_ptr(),
                                 opt_ptr_t<int>(err), stream_of(pos)));
}

// part [768 + 288] f32 (one sequence), latent [cap, 256] / rope [cap, 32] bf16, q_abs [1, H, 288] bf16.
void mla_prep_qb_absorb(const Tensor& part, const Tensor& gamma_q_a, const Tensor& gamma_kv_a, double eps,
                        const Tensor& cos, const Tensor& sin, const Tensor& pos, const Tensor& latent,
                        const Tensor& rope, const Tensor& w_q_b, const Tensor& w_kv_b, const Tensor& q_abs,
                        const OptT& err) {
  need(part, "part", F32);
  const int64_t QL = part.numel() - 288;
  need(gamma_q_a, "gamma_q_a", BF, QL);
  need(gamma_kv_a, "gamma_kv_a", BF, 256);
  need(pos, "pos", I32, 1);
  need(latent, "latent", BF);
  if (latent.dim() < 1 || latent.size(-1) != 256) bad("latent: expected (cap, 256)");
  const int64_t cap = latent.numel() / 256;
  need(rope, "rope", BF, cap * 32);
  need(q_abs, "q_abs", BF);
  if (q_abs.dim() != 3 || q_abs.size(0) != 1 || q_abs.size(2) != 288) bad("q_abs: expected (1, heads, 288)");
  const int64_t H = q_abs.size(1);
  need_mat(w_q_b, "w_q_b", H * 96, QL);
  need_mat(w_kv_b, "w_kv_b", H * 128, 256);
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (cos.numel() % 32 != 0) bad("cos: expected (rows, 32)");
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_mla_prep_qb_absorb(part.data_ptr<float>(), QL, gamma_q_a.data_ptr(), gamma_kv_a.data_ptr(),
                                      (float)eps, cos.data_ptr(), sin.data_ptr(), cos.numel() / 32,
                                      pos.data_ptr<int>(), latent.data_ptr(), rope.data_ptr(), cap,
                                      w_q_b.data_ptr(), w_kv_b.data_ptr(), H, q_abs.data_ptr(), opt_ptr_t<int>(err),
                                      stream_of(pos)));
}

// op [B, ns, H, 256] bf16, mp / lp [B, ns, H] f32.
void mla_attention(const Tensor& q_abs, const Tensor& latent, const Tensor& rope, const Tensor& wr,
                   int64_t split, double scale, const Tensor& op, const Tensor& mp, const Tensor& lp,
                   const OptT& err) {
  need(wr, "wr", I32);
  const int64_t B = wr.numel();
  need(q_abs, "q_abs", BF);
  if (q_abs.dim() != 3 || q_abs.size(0) != B || q_abs.size(2) != 288) bad("q_abs: expected (batch, heads, 288)");
  const int64_t H = q_abs.size(1);
  need(latent, "latent", BF);
  if (latent.dim() != 3 || latent.size(0) != B || latent.size(2) != 256) bad("latent: expected (batch, cap, 256)");
  const int64_t cap = latent.size(1);
  need(rope, "rope", BF, B * cap * 32);
  if (split <= 0 || cap % split != 0) bad("cache capacity must be a multiple of the split");
  const int64_t ns = cap / split;
  need(op, "op", BF, B * ns * H * 256);
  need(mp, "mp", F32, B * ns * H);
  need(lp, "lp", F32, B * ns * H);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_mla_attention(q_abs.data_ptr(), latent.data_ptr(), rope.data_ptr(), wr.data_ptr<int>(), B, H,
                                 cap, split, (float)scale, op.data_ptr(), mp.data_ptr<float>(),
                                 lp.data_ptr<float>(), opt_ptr_t<int>(err), stream_of(wr)));
}

void mla_combine_up(const Tensor& op, const Tensor& mp, const Tensor& lp, const Tensor& wr, int64_t split,
                    const Tensor& w_kv_b, const Tensor& attn) {
  need(wr, "wr", I32);
  const int64_t B = wr.numel();
  need(op, "op", BF);
  if (op.dim() != 4 || op.size(0) != B || op.size(3) != 256) bad("op: expected (batch, splits, heads, 256)");
  const int64_t ns = op.size(1), H = op.size(2);
  need(mp, "mp", F32, B * ns * H);
  need(lp, "lp", F32, B * ns * H);
  need_mat(w_kv_b, "w_kv_b", H * 128, 256);
  need(attn, "attn", BF, B * H * 64);
  raise_status(tfa_mla_combine_up(op.data_ptr(), mp.data_ptr<float>(), lp.data_ptr<float>(), wr.data_ptr<int>(),
                                  ns, split, B, H, ns * split, w_kv_b.data_ptr(), attn.data_ptr(), stream_of(wr)));
}

// part [ks, m, hidden] f32; h_in / h_out / xn [m, hidden] bf16
void rows_norm_scaled(const Tensor& part, const Tensor& h_in, double alpha, const Tensor& h_out, const Tensor& gamma,
                      const Tensor& xn, double eps) {
  need(h_in, "h_in", BF);
  if (h_in.dim() != 2) bad("h_in: expected (m, hidden)");
  const int64_t M = h_in.size(0), H = h_in.size(1);
  need(h_out, "h_out", BF, M * H);
  need(xn, "xn", BF, M * H);
  need(gamma, "gamma", BF, H);
  need(part, "part", F32);
  if (M * H == 0 || part.numel() % (M * H) != 0) bad("part: expected (ks, m, hidden)");
  raise_status(tfa_rows_norm_scaled(part.data_ptr<float>(), part.numel() / (M * H), h_in.data_ptr(), (float)alpha,
                                    h_out.data_ptr(), gamma.data_ptr(), xn.data_ptr(), M, H, (float)eps,
                                    stream_of(xn)));
}

// part [ks, m, n] f32; residual / out [m, n] bf16.
void rows_residual(const Tensor& part, const Tensor& residual, double alpha, const Tensor& out) {
  need(residual, "residual", BF);
  if (residual.dim() != 2) bad("residual: expected (m, n)");
  const int64_t M = residual.size(0), N = residual.size(1);
  need(out, "out", BF, M * N);
  need(part, "part", F32);
  if (part.numel() % (M * N) != 0) bad("part: expected (ks, m, n)");
  raise_status(tfa_rows_residual(part.data_ptr<float>(), part.numel() / (M * N), residual.data_ptr(),
                                 (float)alpha, out.data_ptr(), M, N, stream_of(out)));
}

// ------------------------------------------------------------ prefill
// q / gate: (n, heads, 256) views, k / v: (n, kv_heads, 256) views, each with a
// unit innermost stride (views into the packed qkv projection output allowed);
// out (n, heads*256) contiguous.
void prefill_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& gate,
                       const Tensor& out, double scale) {
  auto view3 = [](const Tensor& t, const char* name) {
    if (!t.defined() || !t.is_cuda()) bad(std::string(name) + ": must be a GPU tensor");
    if (t.scalar_type() != BF) bad(std::string(name) + ": expected bfloat16");
    if (t.dim() != 3 || t.stride(2) != 1) bad(std::string(name) + ": expected a (n, heads, d) view with unit inner stride");
  };
  view3(q, "q");
  view3(k, "k");
  view3(v, "v");
  view3(gate, "gate");
  const int64_t N = q.size(0), HQ = q.size(1), Dh = q.size(2), HKV = k.size(1);
  if (k.size(0) != N || v.size(0) != N || gate.size(0) != N || v.size(1) != HKV || gate.size(1) != HQ ||
      k.size(2) != Dh || v.size(2) != Dh || gate.size(2) != Dh)
    bad("prefill_attention: q/gate (n, heads, d) and k/v (n, kv_heads, d) shapes disagree");
  need(out, "out", BF, N * HQ * Dh);
  raise_status(tfa_prefill_attention(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                                     v.data_ptr(), v.stride(0), v.stride(1), gate.data_ptr(), gate.stride(0),
                                     gate.stride(1), out.data_ptr(), HQ * Dh, N, HQ, HKV, Dh, (float)scale,
                                     stream_of(out)));
}

// a [m, k], b [n, k] (row strides from the tensors), c [m, n]; residual [m, n] optional
void gemm_nt(const Tensor& a, const Tensor& b, const Tensor& c, const OptT& residual) {
  auto mat = [](const Tensor& t, const char* name) {
    if (!t.defined() || !t.is_cuda() || t.scalar_type() != BF || t.dim() != 2 || t.stride(1) != 1)
      bad(std::string(name) + ": expected a bf16 GPU matrix with unit inner stride");
  };
  mat(a, "a");
  mat(b, "b");
  mat(c, "c");
  const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
  if (b.size(1) != K || c.size(0) != M || c.size(1) != N) bad("gemm_nt: shapes disagree");
  const void* r = nullptr;
  int64_t ldr = 0;
  if (residual) {
    mat(*residual, "residual");
    if (residual->size(0) != M || residual->size(1) != N) bad("residual: expected (m, n)");
    r = residual->data_ptr();
    ldr = residual->stride(0);
  }
  raise_status(tfa_gemm_nt(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, a.stride(0), b.stride(0),
                           c.stride(0), r, ldr, stream_of(c)));
}

void qkv_norm_rope(const Tensor& hn, const Tensor& w_qkv, const Tensor& out, int64_t heads, int64_t kv_heads,
                   const Tensor& gamma_q, const Tensor& gamma_k, double eps, const Tensor& cos, const Tensor& sin) {
  need(hn, "hn", BF);
  if (hn.dim() != 2) bad("hn: expected (n, hidden)");
  const int64_t N = hn.size(0), H = hn.size(1), W = (2 * heads + 2 * kv_heads) * 256;
  need_mat(w_qkv, "w_qkv", W, H);
  need(out, "out", BF, N * W);
  need(gamma_q, "gamma_q", BF, 256);
  need(gamma_k, "gamma_k", BF, 256);
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (cos.numel() < N * 64) bad("cos / sin: expected at least (n, 64)");
  raise_status(tfa_qkv_norm_rope(hn.data_ptr(), w_qkv.data_ptr(), out.data_ptr(), N, H, heads, kv_heads, 256,
                                 gamma_q.data_ptr(), gamma_k.data_ptr(), (float)eps, cos.data_ptr(), sin.data_ptr(),
                                 64, stream_of(out)));
}

// ------------------------------------------- prompt prefill (decode model)
// a [m, k], b [n, k] bf16 (row strides from the tensors); c [m, n] f32, or
// [ks, m, n] f32 split-K partials (K split into ks ranges)
void gemm_nt_f32(const Tensor& a, const Tensor& b, const Tensor& c) {
  auto mat = [](const Tensor& t, const char* name, at::ScalarType dt) {
    if (!t.defined() || !t.is_cuda() || t.scalar_type() != dt || t.dim() != 2 || t.stride(1) != 1)
      bad(std::string(name) + ": expected a GPU matrix of the right dtype with unit inner stride");
  };
  mat(a, "a", BF);
  mat(b, "b", BF);
  const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
  if (b.size(1) != K) bad("gemm_nt_f32: shapes disagree");
  if (!c.defined() || !c.is_cuda() || c.scalar_type() != F32 || !c.is_contiguous() || (c.dim() != 2 && c.dim() != 3))
    bad("c: expected a contiguous f32 GPU tensor (m, n) or (ks, m, n)");
  const int64_t ks = c.dim() == 3 ? c.size(0) : 1;
  if (c.size(-2) != M || c.size(-1) != N) bad("gemm_nt_f32: shapes disagree");
  raise_status(tfa_gemm_nt_f32_split(a.data_ptr(), b.data_ptr(), c.data_ptr<float>(), M, N, K, a.stride(0),
                                     b.stride(0), N, ks, stream_of(c)));
}

// gu f32 (rows, 2 * inter) or split-K partials (ks, rows, 2 * inter) with
// interleaved gate / up columns; act bf16 (rows, inter)
void swiglu_pairs(const Tensor& gu, const Tensor& act) {
  if (!gu.defined() || !gu.is_cuda() || gu.scalar_type() != F32 || !gu.is_contiguous() || (gu.dim() != 2 && gu.dim() != 3))
    bad("gu: expected a contiguous f32 (rows, 2 * inter) or (ks, rows, 2 * inter) GPU tensor");
  const int64_t ks = gu.dim() == 3 ? gu.size(0) : 1;
  const int64_t R = gu.size(-2), I = gu.size(-1) / 2;
  need(act, "act", BF, R * I);
  if (gu.size(-1) != 2 * I) bad("gu: odd column count");
  raise_status(tfa_swiglu_pairs_split(gu.data_ptr<float>(), ks, 2 * I, R, I, act.data_ptr(), stream_of(gu)));
}

// qkv f32 (batch * n, ldq) or split-K partials (ks, batch * n, ldq); caches
// (batch, cap, hkv * 128) or (cap, hkv * 128); q_out bf16 (batch * n, hq * 128).
void prefill_qk_rope(const Tensor& qkv, const Tensor& gamma_q, const Tensor& gamma_k, double eps, const Tensor& cos,
                     const Tensor& sin, int64_t batch, int64_t n, int64_t pos0, const Tensor& k_cache,
                     const Tensor& v_cache, const Tensor& q_out, int64_t hq, int64_t hkv) {
  need(qkv, "qkv", F32);
  if ((qkv.dim() != 2 && qkv.dim() != 3) || qkv.size(-2) != batch * n) bad("qkv: expected ([ks,] batch * n, columns)");
  const int64_t ks = qkv.dim() == 3 ? qkv.size(0) : 1;
  need(gamma_q, "gamma_q", BF, 128);
  need(gamma_k, "gamma_k", BF, 128);
  need(cos, "cos", BF);
  need(sin, "sin", BF, cos.numel());
  if (cos.dim() != 2 || cos.size(1) != 128) bad("cos / sin: expected (rows, 128)");
  need(k_cache, "k_cache", BF);
  need(v_cache, "v_cache", BF, k_cache.numel());
  const int64_t KN = hkv * 128;
  if (batch < 1 || KN < 1 || k_cache.size(-1) != KN || k_cache.numel() % (batch * KN) != 0)
    bad("k_cache / v_cache: expected (batch, cap, kv_heads * 128)");
  need(q_out, "q_out", BF, batch * n * hq * 128);
  raise_status(tfa_prefill_qk_rope_split(qkv.data_ptr<float>(), ks, qkv.size(-1), gamma_q.data_ptr(), gamma_k.data_ptr(),
                                   (float)eps, cos.data_ptr(), sin.data_ptr(), cos.size(0), batch, n, pos0,
                                   k_cache.data_ptr(), v_cache.data_ptr(), k_cache.numel() / (batch * KN),
                                   q_out.data_ptr(), hq, hkv, 128, stream_of(qkv)));
}

// q (batch, n, heads, d), k / v (batch, >= n, kv_heads, d) views with unit inner
// stride (the decode cache viewed in place); out (batch, n, heads * d) with a
// unit inner stride.
void causal_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out, double scale) {
  auto view4 = [](const Tensor& t, const char* name) {
    if (!t.defined() || !t.is_cuda()) bad(std::string(name) + ": must be a GPU tensor");
    if (t.scalar_type() != BF) bad(std::string(name) + ": expected bfloat16");
    if (t.dim() != 4 || t.stride(3) != 1) bad(std::string(name) + ": expected a (batch, n, heads, d) view with unit inner stride");
  };
  view4(q, "q");
  view4(k, "k");
  view4(v, "v");
  const int64_t B = q.size(0), N = q.size(1), HQ = q.size(2), Dh = q.size(3), HKV = k.size(2);
  if (k.size(0) != B || v.size(0) != B || k.size(1) < N || v.size(1) < N || v.size(2) != HKV || k.size(3) != Dh ||
      v.size(3) != Dh)
    bad("causal_attention: q (batch, n, heads, d) and k/v (batch, >= n, kv_heads, d) shapes disagree");
  if (!out.defined() || !out.is_cuda() || out.scalar_type() != BF || out.dim() != 3 || out.size(0) != B ||
      out.size(1) != N || out.size(2) != HQ * Dh || out.stride(2) != 1)
    bad("out: expected a bf16 (batch, n, heads * d) GPU tensor with unit inner stride");
  raise_status(tfa_causal_attention(q.data_ptr(), q.stride(1), q.stride(2), q.stride(0), k.data_ptr(), k.stride(1),
                                    k.stride(2), k.stride(0), v.data_ptr(), v.stride(1), v.stride(2), v.stride(0),
                                    out.data_ptr(), out.stride(1), out.stride(0), B, N, HQ, HKV, Dh, (float)scale,
                                    stream_of(out)));
}

// ------------------------------------------------- per-op decode entries
void rmsnorm_gemv_gate_up(const Tensor& h, const Tensor& gamma, double eps, const Tensor& w_gate,
                          const Tensor& w_up, const Tensor& act) {
  need(h, "x", BF);
  const int64_t K = h.numel();
  need(gamma, "gamma", BF, K);
  const int64_t I = act.numel();
  need_mat(w_gate, "w_gate", I, K);
  need_mat(w_up, "w_up", I, K);
  need(act, "out", BF, I);
  raise_status(tfa_rmsnorm_gemv_gate_up(h.data_ptr(), gamma.data_ptr(), (float)eps,
                                        w_gate.data_ptr(), w_up.data_ptr(), act.data_ptr(), I, K,
                                        stream_of(h)));
}

void lm_head_gemv(const Tensor& h, const Tensor& w, double divisor, const Tensor& logits) {
  need(h, "hidden", BF);
  const int64_t K = h.numel();
  if (w.dim() != 2) bad("w_head: expected a 2-D (vocab, hidden) weight");
  const int64_t V = w.size(0);
  need_mat(w, "w_head", V, K);
  need(logits, "out", BF, V);
  raise_status(tfa_lm_head_gemv(h.data_ptr(), w.data_ptr(), (float)divisor, logits.data_ptr(), V, K,
                                stream_of(h)));
}

void silu_mul(const Tensor& part, const Tensor& act) {
  need(part, "P", F32);
  need(act, "O", BF);
  if (part.dim() != 2 && part.dim() != 3) bad("P: expected (SK, [rows,] 2I)");
  const int64_t rows = part.dim() == 3 ? part.size(1) : 1;
  const int64_t I = part.size(-1) / 2;
  if (part.size(-1) != 2 * I || act.numel() != rows * I) bad("P / O: expected P (SK, [rows,] 2I) and O (rows, I)");
  raise_status(tfa_silu_mul(part.data_ptr<float>(), part.size(0), I, rows, act.data_ptr(),
                            stream_of(part)));
}

void embed(const Tensor& table, const Tensor& ids, const Tensor& out, const std::optional<double>& scale,
           const OptT& err) {
  need(table, "table", BF);
  if (table.dim() != 2) bad("table: expected (vocab, hidden)");
  need(ids, "ids", I64);
  const int64_t rows = ids.numel();
  need(out, "out", BF, rows * table.size(1));
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_embed(table.data_ptr(), ids.data_ptr<int64_t>(), table.size(0), table.size(1),
                         rows, scale ? 1 : 0, scale ? (float)*scale : 1.f, out.data_ptr(),
                         opt_ptr_t<int>(err), stream_of(table)));
}

void qk_rope_cache(const Tensor& part, const Tensor& gamma_q, const Tensor& gamma_k, double eps,
                   const Tensor& cos_t, const Tensor& sin_t, const Tensor& pos, const Tensor& wr,
                   const Tensor& k_cache, const Tensor& v_cache, const Tensor& q_out, int64_t hq,
                   int64_t hkv, const OptT& err) {
  const int64_t D = 128;
  need(pos, "Pos", I32);
  const int64_t B = pos.numel();
  need(wr, "Wr", I32, B);
  need(part, "P", F32);
  const int64_t per = B * (hq + 2 * hkv) * D;
  if (part.numel() % per != 0) bad("P: expected (SK, [batch,] (HQ + 2 HKV) * 128)");
  need(gamma_q, "Gq", BF, D);
  need(gamma_k, "Gk", BF, D);
  need(cos_t, "Cos", BF);
  need(sin_t, "Sin", BF, cos_t.numel());
  if (cos_t.dim() != 2 || cos_t.size(1) != D) bad("Cos: expected (MP, 128)");
  need(k_cache, "Kc", BF);
  need(v_cache, "Vc", BF, k_cache.numel());
  if (k_cache.numel() % (B * hkv * D) != 0) bad("Kc: size is not a multiple of batch*HKV*128");
  const int64_t cap = k_cache.numel() / (B * hkv * D);
  need(q_out, "Q", BF, B * hq * D);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_qk_rope_cache(part.data_ptr<float>(), part.numel() / per, gamma_q.data_ptr(),
                                 gamma_k.data_ptr(), (float)eps, cos_t.data_ptr(), sin_t.data_ptr(),
                                 cos_t.size(0), pos.data_ptr<int>(), wr.data_ptr<int>(),
                                 k_cache.data_ptr(), v_cache.data_ptr(), cap, q_out.data_ptr(), B, hq,
                                 hkv, D, opt_ptr_t<int>(err), stream_of(part)));
}

void attn_combine_gemv_residual(const Tensor& op, const Tensor& mp, const Tensor& lp, const OptT& wr, int64_t split,
                                const Tensor& w_o, const Tensor& residual, const Tensor& y, const OptT& attn_out) {
  const int64_t D = 128;
  need(mp, "Mp", F32);
  if (mp.dim() != 2) bad("Mp: expected (NS, HQ)");
  const int64_t ns = mp.size(0), hq = mp.size(1);
  need(op, "Op", F32, ns * hq * D);
  need(lp, "Lp", F32, ns * hq);
  if (wr) need(*wr, "wr", I32, 1);
  if (w_o.dim() != 2) bad("w_o: expected a 2-D (N, HQ*128) weight");
  const int64_t N = w_o.size(0);
  need_mat(w_o, "w_o", N, hq * D);
  need(residual, "residual", BF, N);
  need(y, "y", BF, N);
  if (attn_out) need(*attn_out, "attn_out", BF, hq * D);
  raise_status(tfa_attn_combine_gemv_residual(op.data_ptr<float>(), mp.data_ptr<float>(), lp.data_ptr<float>(), ns,
                                              hq, D, opt_ptr_t<const int>(wr), split, w_o.data_ptr(),
                                              residual.data_ptr(), y.data_ptr(), N, opt_ptr_t<void>(attn_out),
                                              stream_of(op)));
}

void decode_attention_seq(const Tensor& part, const Tensor& gamma_q, const Tensor& gamma_k, double eps,
                          const Tensor& cos_t, const Tensor& sin_t, const Tensor& pos, const Tensor& wr,
                          const Tensor& k_cache, const Tensor& v_cache, int64_t hq, int64_t hkv, double scale,
                          const Tensor& out, const OptT& err) {
  const int64_t D = 128;
  need(pos, "Pos", I32);
  const int64_t B = pos.numel();
  need(wr, "Wr", I32, B);
  need(part, "P", F32);
  const int64_t per = B * (hq + 2 * hkv) * D;
  if (part.numel() % per != 0) bad("P: expected (SK, [batch,] (HQ + 2 HKV) * 128)");
  need(gamma_q, "Gq", BF, D);
  need(gamma_k, "Gk", BF, D);
  need(cos_t, "Cos", BF);
  need(sin_t, "Sin", BF, cos_t.numel());
  if (cos_t.dim() != 2 || cos_t.size(1) != D) bad("Cos: expected (MP, 128)");
  need(k_cache, "Kc", BF);
  need(v_cache, "Vc", BF, k_cache.numel());
  if (k_cache.numel() % (B * hkv * D) != 0) bad("Kc: size is not a multiple of batch*HKV*128");
  const int64_t cap = k_cache.numel() / (B * hkv * D);
  need(out, "O", BF, B * hq * D);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_decode_attention_seq(part.data_ptr<float>(), part.numel() / per, gamma_q.data_ptr(),
                                        gamma_k.data_ptr(), (float)eps, cos_t.data_ptr(), sin_t.data_ptr(),
                                        cos_t.size(0), k_cache.data_ptr(), v_cache.data_ptr(),
                                        pos.data_ptr<int>(), wr.data_ptr<int>(), B, hq, hkv, D, cap,
                                        (float)scale, out.data_ptr(), opt_ptr_t<int>(err), stream_of(part)));
}

void rope_attend(const Tensor& q_up, const Tensor& kv_up, const Tensor& k_rope, const Tensor& cos_t,
                 const Tensor& sin_t, const Tensor& pos, const Tensor& k_cache, const Tensor& v_cache,
                 const Tensor& ctx, const Tensor& scale, int64_t heads, int64_t nope, int64_t rope,
                 int64_t v_dim, const Tensor& op, const Tensor& mp, const Tensor& lp, const Tensor& attn,
                 const OptT& k_new, const OptT& v_new, const OptT& err) {
  const int64_t qk = nope + rope;
  need(q_up, "q_up", BF, heads * qk);
  need(kv_up, "kv_up", BF, heads * (nope + v_dim));
  need(k_rope, "k_rope", BF, rope);
  need(cos_t, "cos", BF);
  need(sin_t, "sin", BF, cos_t.numel());
  if (cos_t.dim() != 2 || cos_t.size(1) != rope) bad("cos: expected (rows, rope)");
  need(pos, "pos", I32, 1);
  need(ctx, "ctx", I32, 1);
  need(scale, "scale", BF, 1);
  need(k_cache, "k_cache", BF);
  if (k_cache.numel() % (heads * qk) != 0) bad("k_cache: expected (capacity, heads, nope + rope)");
  const int64_t cap = k_cache.numel() / (heads * qk);
  need(v_cache, "v_cache", BF, cap * heads * v_dim);
  const int64_t ns = tfa_rope_attend_splits(cap);
  need(op, "op", F32, ns * heads * v_dim);
  need(mp, "mp", F32, ns * heads);
  need(lp, "lp", F32, ns * heads);
  need(attn, "attn", BF, heads * v_dim);
  if (k_new) need(*k_new, "k_new", BF, heads * qk);
  if (v_new) need(*v_new, "v_new", BF, heads * v_dim);
  if (err) need(*err, "err", I32, 1);
  raise_status(tfa_rope_attend(
      q_up.data_ptr(), kv_up.data_ptr(), k_rope.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(),
      cos_t.size(0), pos.data_ptr<int>(), cap ? k_cache.data_ptr() : nullptr,
      cap ? v_cache.data_ptr() : nullptr, cap, ctx.data_ptr<int>(), scale.data_ptr(), heads, nope,
      rope, v_dim, ns ? op.data_ptr<float>() : nullptr, ns ? mp.data_ptr<float>() : nullptr,
      ns ? lp.data_ptr<float>() : nullptr, attn.data_ptr(), opt_ptr(k_new) ? k_new->data_ptr() : nullptr,
      opt_ptr(v_new) ? v_new->data_ptr() : nullptr, opt_ptr_t<int>(err), stream_of(q_up)));
}

void copy_stream(const Tensor& src, const Tensor& dst) {
  if (!src.is_cuda() || !dst.is_cuda() || !src.is_contiguous() || !dst.is_contiguous())
    bad("copy_stream: contiguous GPU tensors required");
  const int64_t nbytes = src.numel() * src.element_size();
  if (dst.numel() * dst.element_size() != nbytes) bad("copy_stream: size mismatch");
  raise_status(tfa_copy_stream(src.data_ptr(), dst.data_ptr(), nbytes, stream_of(src)));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "tilefoundry_amd: thin torch bindings over the gfx950 C ABI";
  m.def("abi_version", &tfa_abi_version);
  m.def("rms_norm", &rms_norm);
  m.def("rms_norm_div", &rms_norm_div);
  m.def("add_rms_norm", &add_rms_norm);
  m.def("resid_rms_norm_partials", &resid_rms_norm_partials);
  m.def("gemv", &gemv);
  m.def("rmsnorm_gemv", &rmsnorm_gemv);
  m.def("rmsnorm_gemv_f32", &rmsnorm_gemv_f32);
  m.def("gemv_residual", &gemv_residual);
  m.def("rmsnorm_gemv_swiglu", &rmsnorm_gemv_swiglu);
  m.def("lm_head_blocks", [](int64_t vocab) { return tfa_lm_head_blocks(vocab); });
  m.def("lm_head_argmax", &lm_head_argmax);
  m.def("sample_step", &sample_step);
  m.def("decode_qkv", &decode_qkv);
  m.def("decode_attention", &decode_attention);
  m.def("attn_combine", &attn_combine);
  m.def("copy_stream", &copy_stream);
  m.def("read_rows", [](const Tensor& w, int64_t rows_per_block, const Tensor& out) {
    if (!w.is_cuda() || !w.is_contiguous() || w.scalar_type() != at::kBFloat16 || w.dim() != 2)
      bad("read_rows: contiguous bf16 GPU matrix required");
    need(out, "out", F32, (w.size(0) + rows_per_block - 1) / std::max<int64_t>(rows_per_block, 1));
    raise_status(tfa_read_rows(w.data_ptr(), w.size(0), w.size(1), rows_per_block, out.data_ptr<float>(),
                               stream_of(w)));
  });
  m.def("skinny_blocks", [](int64_t n) { return tfa_skinny_blocks(n); });
  m.def("skinny_gemm", &skinny_gemm);
  m.def("rows_norm", &rows_norm);
  m.def("batch_sample_step", &batch_sample_step);
  m.def("top_p_sample_step", &top_p_sample_step);
  m.def("skinny_gemm_residual", &skinny_gemm_residual);
  m.def("skinny_gemm_norm_swiglu", &skinny_gemm_norm_swiglu);
  m.def("skinny_residual_blocks", [](int64_t n) { return tfa_skinny_residual_blocks(n); });
  m.def("mla_prep", &mla_prep);
  m.def("mla_prep_q_gemv", &mla_prep_q_gemv);
  m.def("mla_q_absorb", &mla_q_absorb);
  m.def("mla_qb_absorb", &mla_qb_absorb);
  m.def("mla_prep_qb_absorb", &mla_prep_qb_absorb);
  m.def("mla_attention", &mla_attention);
  m.def("mla_combine_up", &mla_combine_up);
  m.def("rows_residual", &rows_residual);
  m.def("rows_norm_scaled", &rows_norm_scaled);
  m.def("prefill_attention", &prefill_attention);
  m.def("gemm_nt", &gemm_nt);
  m.def("qkv_norm_rope", &qkv_norm_rope);
  m.def("gemm_nt_f32", &gemm_nt_f32);
  m.def("gemm_f32_splits", [](int64_t m, int64_t n, int64_t k) { return tfa_gemm_f32_splits(m, n, k); });
  m.def("swiglu_pairs", &swiglu_pairs);
  m.def("prefill_qk_rope", &prefill_qk_rope);
  m.def("causal_attention", &causal_attention);
  m.def("rmsnorm_gemv_gate_up", &rmsnorm_gemv_gate_up);
  m.def("lm_head_gemv", &lm_head_gemv);
  m.def("silu_mul", &silu_mul);
  m.def("embed", &embed);
  m.def("qk_rope_cache", &qk_rope_cache);
  m.def("decode_attention_seq", &decode_attention_seq);
  m.def("attn_combine_gemv_residual", &attn_combine_gemv_residual);
  m.def("rope_attend_splits", [](int64_t cap) { return tfa_rope_attend_splits(cap); });
  m.def("rope_attend", &rope_attend);
}
