// Decode GEMVs for weights stored [N, K] (out, in), plus the greedy pick.
//
// gemv_rows: y[n] = sum_k x[k] W[n, k]. A 256-thread block owns R consecutive
// rows; its four waves split K into contiguous quarters, so each wave reads a
// contiguous 1 KB run of a row per load instruction (16 bytes a lane) and the
// block reads R whole rows back to back. The input vector (and the norm scale)
// is issued first -- it is L2-resident and its round trip should not queue
// behind the weights -- then every weight load of the block, then the prologue
// math runs while the weights are in flight. The R partial dots of a wave are
// reduced by one transposed butterfly and the four waves meet in LDS in wave
// order, so the result does not depend on scheduling. No block depends on
// another: there is no in-kernel handshake (on gfx950 each one costs a few
// coherent memory round trips, more than a kernel boundary).
//
// Prologues:  plain x | rmsnorm(h) | rmsnorm(embed[ids[0]])
// Epilogues:  f32 | bf16 | residual add | scaled residual add | SwiGLU pair |
//             q|k rows to a bf16 buffer and v rows into the KV cache slot |
//             logits + the block's best (value, lowest index)
// The greedy pick over the block winners is a one-block kernel of its own.
//
// Reference kernels replaced: examples/qwen3_1_7b-tilelang/fast/kernels.py
// (rms_norm :58-79, gemv :123-145, gemv_silu :210-257, lm_head :260-321, embed
// :579-588, sample_step :591-637) and the MiniCPM3 GEMVs
// examples/minicpm3_4b-cutedsl/kernels/cute_gemv.py:246-495.
#include <float.h>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kLmHeadRows = 16;  // rows per block of the head (one argmax candidate each)

enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_EMBED_NORM = 2, PRO_LORA = 3 };
constexpr int kLoraLat = 256;   // MLA latent width (kv_lora_rank)
constexpr int kLoraRope = 32;   // MLA rope slice
enum {
  EPI_F32 = 0, EPI_BF16 = 1, EPI_RESID = 2, EPI_RESID_SCALED = 3, EPI_SWIGLU = 4,
  EPI_ARGMAX = 5, EPI_QKV = 6
};

struct GemvArgs {
  // input vector
  const uint16_t* x;      // [K] bf16: the vector (plain) or the row to normalise
  const uint16_t* gamma;  // [K] norm scale
  const uint16_t* table;  // [V, K] embedding table (embed prologue)
  const int64_t* ids;     // [1] token id (embed prologue)
  uint16_t* h_copy;       // [K] gathered row, written by block 0 (embed prologue)
  int64_t vocab;          // rows of `table`
  float eps;
  // matrix
  const uint16_t* w;      // [N, K]
  const uint16_t* w_odd;  // SwiGLU from separate matrices: odd rows 2i+1 are w_odd[i], even rows w[i]
  int N, K;
  float in_div;           // plain prologue: x lands as bf16(x / in_div) when nonzero
  // outputs
  float* yf;              // f32 out / logits
  uint16_t* yb;           // bf16 out (also the q|k rows of the qkv routing)
  const uint16_t* res;    // [N] residual
  const uint16_t* alpha;  // [1] bf16 residual scale
  float* bv;              // [gridDim.x] block maxima (argmax)
  int* bi;                // [gridDim.x] their indices
  // qkv routing: rows >= n_qk are value rows, written to vc[wr[0], :]
  int n_qk;
  const int* wr;
  int cap;
  uint16_t* vc;
  int* err;
  // LoRA prologue (MLA at one sequence): xf = [q_a (K) | kv_c (256) | k_rope (32)]
  // f32, one split; block 0 also lands the latent and rope key at pos[0].
  const float* xf;
  const uint16_t* gkv;    // [256] latent norm scale
  const uint16_t* cos_t;  // [rope_rows, 32]
  const uint16_t* sin_t;
  int rope_rows;
  const int* pos;
  uint16_t* lat_cache;    // [cap, 256]
  uint16_t* rope_cache;   // [cap, 32]
};

TFA_DEV void set_err(int* err, int code) {
  if (err) atomicExch(err, code);
}

// (value, index) order for greedy argmax: larger value wins, equal values go to
// the lower index (torch.argmax), NaN never wins.
TFA_DEV bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

template <int NCH, int R, int PRO, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_rows_kernel(const GemvArgs a) {
  __shared__ float red[kWaves][R];
  __shared__ float ssq[kWaves];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int t = threadIdx.x;
  const int row0 = blockIdx.x * R;
  const int K = a.K;
  const int kq = K / kWaves;   // elements in this wave's quarter
  const int nch = kq >> 3;     // 16-byte chunks in the quarter
  const int kbase = wid * kq;

  // 1. the input vector's quarter and its norm scale
  const uint16_t* src = a.x;
  if (PRO == PRO_EMBED_NORM) {
    int64_t id = a.ids[0];
    if (id < 0 || id >= a.vocab) {
      if (blockIdx.x == 0 && t == 0) set_err(a.err, 1);
      id = 0;
    }
    src = a.table + id * K;
  }
  uint4 xv[NCH], gv[NCH];
  // LoRA prologue: q_a[t + 256 j] (the order its norm sums in), this lane's f32
  // chunks, and for block 0 the latent column t, the rope slice and the position
  float qs[4], xl[NCH][8];
  float cv = 0.f, krv = 0.f;
  int p_raw = 0;
  const bool side = PRO == PRO_LORA && blockIdx.x == 0;
  uint32_t gkr = 0, cr = 0, sr = 0;
  if (PRO == PRO_LORA) {
    // unconditional loads at clamped indices (values past the shape are zeroed
    // once landed); every block also loads block 0's latent / rope operands
    // (a few hundred bytes from L2) so that no load sits behind a branch; the
    // position first, so the rope row can follow without waiting for the rest
    p_raw = a.pos[0];
#pragma unroll
    for (int j = 0; j < 4; ++j) qs[j] = a.xf[min(t + kThreads * j, K - 1)];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = min(lane + j * kWave, nch - 1);
      const float4 lo = __builtin_bit_cast(float4, ld16(a.xf + kbase + 8 * c));
      const float4 hi = __builtin_bit_cast(float4, ld16(a.xf + kbase + 8 * c + 4));
      xl[j][0] = lo.x; xl[j][1] = lo.y; xl[j][2] = lo.z; xl[j][3] = lo.w;
      xl[j][4] = hi.x; xl[j][5] = hi.y; xl[j][6] = hi.z; xl[j][7] = hi.w;
      gv[j] = ld16(a.gamma + kbase + 8 * c);
    }
    gkr = a.gkv[t];
    cv = a.xf[K + t];
    krv = a.xf[K + kLoraLat + min(t, kLoraRope - 1)];
    const bool pv = p_raw >= 0 && p_raw < a.cap && p_raw < a.rope_rows;
    const size_t ro = static_cast<size_t>(pv ? p_raw : 0) * kLoraRope + min(t, kLoraRope - 1);
    cr = a.cos_t[ro];
    sr = a.sin_t[ro];
  } else {
    // unconditional (a chunk past the quarter reads its last chunk, zeroed once
    // landed): no load behind a branch, so the norm below waits for these alone
    // and not for the weights issued after them
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = min(lane + j * kWave, nch - 1);
      xv[j] = ld16(src + kbase + 8 * c);
      if (PRO != PRO_PLAIN) gv[j] = ld16(a.gamma + kbase + 8 * c);
    }
  }

  // the epilogue's own inputs (the residual row, the residual scale, the value
  // cache slot) go out with the first loads, so the epilogue adds no round trip
  uint32_t res_raw = 0, al_raw = 0;
  int slot_raw = 0;
  if constexpr (EPI == EPI_RESID || EPI == EPI_RESID_SCALED)
    res_raw = a.res[min(row0 + min(t, R - 1), a.N - 1)];
  if constexpr (EPI == EPI_RESID_SCALED) al_raw = a.alpha[0];
  if constexpr (EPI == EPI_QKV) slot_raw = a.wr[0];

  // 2. weights: streamed once, non-temporal
  uint4 w[R][NCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + j * kWave;
      // R is even, so (row & 1) == (r & 1) and the matrix pick is static
      // rows past N and chunks past the quarter read the last ones (real, finite
      // weights): the chunk's input is zero and the row is never stored
      const int rc = min(row, a.N - 1);
      const uint16_t* wrow = (EPI == EPI_SWIGLU && a.w_odd)
                                 ? ((r & 1) ? a.w_odd : a.w) + static_cast<size_t>(rc >> 1) * K
                                 : a.w + static_cast<size_t>(rc) * K;
      w[r][j] = ld16_stream(wrow + kbase + 8 * min(c, nch - 1));
    }
  }

  // 3. prologue math while the weights are in flight
  if (PRO == PRO_EMBED_NORM && blockIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + j * kWave;
      if (c < nch) st16(a.h_copy + kbase + 8 * c, xv[j]);
    }
  }
  float xf[NCH][8];
  if (PRO != PRO_LORA) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) unpack8(lane + j * kWave < nch ? xv[j] : make_uint4(0, 0, 0, 0), xf[j]);
  }
  if (PRO == PRO_PLAIN && a.in_div != 0.f) {
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) xf[j][i] = round_bf(__fdiv_rn(xf[j][i], a.in_div));
  }
  if (PRO == PRO_LORA) {
    // Each projection value lands in bf16 (a one-split sum, 0 + v); the q_a norm
    // sums thread t's values j = 0..3, then the wave, then waves 0..3 in order, and
    // block 0 reduces the latent's squares alongside.
    __shared__ float kss[kWaves];
    __shared__ float kr[kLoraRope];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q = round_bf(0.f + (t + kThreads * j < K ? qs[j] : 0.f));
      ss += q * q;
    }
    ss = wave_sum(ss);
    float sk = 0.f, c = 0.f, s = 0.f;
    bool p_ok = false;
    if (side) {
      cv = round_bf(0.f + cv);
      sk = wave_sum(cv * cv);
      if (t < kLoraRope) kr[t] = round_bf(0.f + krv);
      p_ok = p_raw >= 0 && p_raw < a.cap && p_raw < a.rope_rows;
      if (t < kLoraRope && p_ok) {
        c = bf2f(cr);
        s = bf2f(sr);
      }
    }
    if (lane == 0) {
      ssq[wid] = ss;
      kss[wid] = sk;
    }
    lds_barrier();   // also publishes kr
    float tq = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tq += ssq[w];
    const float rq = rsqrt_rn(tq / static_cast<float>(K) + a.eps);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float g[8];
      unpack8(gv[j], g);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        xf[j][i] = lane + j * kWave < nch ? round_bf(round_bf(round_bf(0.f + xl[j][i]) * rq) * g[i]) : 0.f;
    }
    if (side) {
      float tk = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) tk += kss[w];
      const float rk = rsqrt_rn(tk / static_cast<float>(kLoraLat) + a.eps);
      if (!p_ok) {
        if (t == 0) set_err(a.err, 6);
      } else {
        a.lat_cache[static_cast<size_t>(p_raw) * kLoraLat + t] =
            static_cast<uint16_t>(f2bf(round_bf(cv * rk) * bf2f(gkr)));
        if (t < kLoraRope) {
          const float x = kr[t];
          const float partner = t < kLoraRope / 2 ? -kr[t + kLoraRope / 2] : kr[t - kLoraRope / 2];
          a.rope_cache[static_cast<size_t>(p_raw) * kLoraRope + t] =
              static_cast<uint16_t>(f2bf(round_bf(round_bf(x * c) + round_bf(partner * s))));
        }
      }
    }
  }
  if (PRO == PRO_NORM || PRO == PRO_EMBED_NORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += xf[j][i] * xf[j][i];
    ss = wave_sum(ss);
    if (lane == 0) ssq[wid] = ss;
    lds_barrier();
    const float tot = (ssq[0] + ssq[1]) + (ssq[2] + ssq[3]);
    const float rs = rsqrt_rn(tot / static_cast<float>(K) + a.eps);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float g[8];
      unpack8(gv[j], g);
#pragma unroll
      for (int i = 0; i < 8; ++i) xf[j][i] = round_bf(round_bf(xf[j][i] * rs) * g[i]);
    }
  }

  // 4. dots, then one transposed reduction for all R rows of the wave
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float f[8];
      unpack8(w[r][j], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) s = fmaf(xf[j][i], f[i], s);
    }
    acc[r] = s;
  }
  {
    const float tot = wave_sum_rows<R>(acc, lane);
    if ((lane & (kWave / R - 1)) == 0) red[wid][wave_rows_owner<R>(lane)] = tot;
  }
  lds_barrier();
  auto total = [&](int r) { return (red[0][r] + red[1][r]) + (red[2][r] + red[3][r]); };

  // 5. epilogues
  if (EPI == EPI_F32 || EPI == EPI_BF16 || EPI == EPI_RESID || EPI == EPI_RESID_SCALED) {
    if (t < R && row0 + t < a.N) {
      const int row = row0 + t;
      const float v = total(t);
      if (EPI == EPI_F32) a.yf[row] = v;
      if (EPI == EPI_BF16) a.yb[row] = static_cast<uint16_t>(f2bf(v));
      if (EPI == EPI_RESID) a.yb[row] = static_cast<uint16_t>(f2bf(__uint_as_float(res_raw << 16) + round_bf(v)));
      if (EPI == EPI_RESID_SCALED) {
        const float al = __uint_as_float(al_raw << 16);
        a.yb[row] = static_cast<uint16_t>(f2bf(__uint_as_float(res_raw << 16) + round_bf(round_bf(v) * al)));
      }
    }
  }
  if (EPI == EPI_SWIGLU) {
    // rows (2i, 2i+1) are (gate_i, up_i):  act_i = bf16(bf16(silu(bf16 g)) * bf16 u)
    if (t < R / 2 && row0 + 2 * t + 1 < a.N) {
      const float g = round_bf(total(2 * t));
      const float u = round_bf(total(2 * t + 1));
      const float act = round_bf(round_bf(g / (1.0f + expf(-g))) * u);
      a.yb[row0 / 2 + t] = static_cast<uint16_t>(f2bf(act));
    }
  }
  if (EPI == EPI_QKV) {
    if (t < R && row0 + t < a.N) {
      const int row = row0 + t;
      const uint16_t v = static_cast<uint16_t>(f2bf(total(t)));
      if (row < a.n_qk) {
        a.yb[row] = v;
      } else {
        const int slot = slot_raw;
        const int nv = a.N - a.n_qk;  // value row width (hkv * head_dim)
        if (slot < 0 || slot >= a.cap) set_err(a.err, 3);
        else a.vc[static_cast<size_t>(slot) * nv + (row - a.n_qk)] = v;
      }
    }
  }
  if (EPI == EPI_ARGMAX) {
    if (t < R && row0 + t < a.N) a.yf[row0 + t] = total(t);
    if (t == 0) {
      float bvv = -FLT_MAX;
      int bii = row0;
      bool any = false;
      for (int r = 0; r < R && row0 + r < a.N; ++r) {
        const float v = total(r);
        if (!any || better(v, row0 + r, bvv, bii)) { bvv = v; bii = row0 + r; any = true; }
      }
      a.bv[blockIdx.x] = bvv;
      a.bi[blockIdx.x] = bii;
    }
  }
}

template <int NCH, int R, int PRO, int EPI>
int launch_gemv(const GemvArgs& a, hipStream_t s, const char* name) {
  const int blocks = (a.N + R - 1) / R;
  gemv_rows_kernel<NCH, R, PRO, EPI><<<blocks, kThreads, 0, s>>>(a);
  return launched(name);
}

// Chunks per lane for one wave's quarter of K.
int chunks_for(int K) { return (K / kWaves / 8 + kWave - 1) / kWave; }

template <int R, int PRO, int EPI>
int dispatch_k(const GemvArgs& a, hipStream_t s, const char* name) {
  switch (chunks_for(a.K)) {
    case 1: return launch_gemv<1, R, PRO, EPI>(a, s, name);
    case 2: return launch_gemv<2, R, PRO, EPI>(a, s, name);
    case 3: return launch_gemv<3, R, PRO, EPI>(a, s, name);
    case 4: return launch_gemv<4, R, PRO, EPI>(a, s, name);
    default: return fail(TFA_ERR_SHAPE, "%s: K=%d exceeds 8192", name, a.K);
  }
}

// Rows per block: enough blocks to cover 256 CUs a few times over. Measured on
// the decode steps' shapes: 2 rows up to 2560 rows (Qwen3 o_proj 3.75 -> 3.64 us,
// down 6.16 -> 6.02 us; MiniCPM3's 2560-row o_proj and down likewise), 4 up to
// 16383 (q|k|v 4096 x 2048: 5.73 -> 5.61 us against 8 rows; gate|up 12288 x
// 2048 the same at 4 or 8), 8 beyond.
template <int PRO, int EPI>
int dispatch_rows(const GemvArgs& a, hipStream_t s, const char* name) {
  if (a.N >= 16384 && a.K <= 4096) return dispatch_k<8, PRO, EPI>(a, s, name);
  if (a.N <= 2560) return dispatch_k<2, PRO, EPI>(a, s, name);
  return dispatch_k<4, PRO, EPI>(a, s, name);
}

int check_gemv(const GemvArgs& a, const char* name) {
  if (a.K <= 0 || a.K % 32 != 0 || a.K > 8192)
    return fail(TFA_ERR_SHAPE, "%s: K=%d must be a positive multiple of 32, at most 8192", name, a.K);
  if (a.N <= 0) return fail(TFA_ERR_SHAPE, "%s: N=%d must be positive", name, a.N);
  if (!a.w) return fail(TFA_ERR_NULL, "%s: null weight", name);
  if (!aligned16(a.w)) return fail(TFA_ERR_ALIGN, "%s: weight not 16-byte aligned", name);
  return TFA_OK;
}

int check_vec(const void* p, const char* what, const char* name) {
  if (!p) return fail(TFA_ERR_NULL, "%s: null %s", name, what);
  if (!aligned16(p)) return fail(TFA_ERR_ALIGN, "%s: %s not 16-byte aligned", name, what);
  return TFA_OK;
}

#define TFA_TRY(expr) do { int _st = (expr); if (_st != TFA_OK) return _st; } while (0)

// Final greedy pick over the head's block winners, then the sample step:
// record the pick at pos, feed the next prompt id while the prompt lasts (else
// the pick), advance pos. One block; ties go to the lowest index.
constexpr int kSampleThreads = 1024;

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(
    const float* __restrict__ bv, const int* __restrict__ bi, int nb, const int* inp,
    const int* plen, int64_t* ids, int* pos, int* sam, int nsteps, int* err) {
  __shared__ float rv[kSampleThreads / kWave];
  __shared__ int ri[kSampleThreads / kWave];
  const int t = threadIdx.x;
  // the position and prompt length first, the next prompt id as soon as the
  // position is known: none of them waits behind the candidates' round trip
  const int p = pos[0];
  const int pl = plen[0];
  int nxt = 0;
  auto next_id = [&]() { nxt = inp[min(max(p + 1, 0), nsteps - 1)]; };
  int best;
  if (nb <= 16 * kSampleThreads) {
    best = block_best_once<16>(bv, bi, nb, rv, ri, next_id);
  } else {
    next_id();
    best = block_best(bv, bi, nb, rv, ri);
  }
  if (t == 0) {
    if (p < 0 || p >= nsteps) {
      set_err(err, 2);
    } else {
      sam[p] = best;
      const bool prompt = (p + 1 < pl) && (p + 1 < nsteps);
      ids[0] = prompt ? static_cast<int64_t>(nxt) : static_cast<int64_t>(best);
      pos[0] = p + 1;
    }
  }
}

// SwiGLU over split-K partials [ks, rows, 2 * inter] of a fused gate|up
// projection (gate in [0, inter), up in [inter, 2 inter)):
//   act[r, i] = bf16(bf16(silu(bf16 g)) * bf16 u), g and u summed in split order.
// examples/qwen3_1_7b-tilelang/fast/kernels.py:547-572 (silu_mul).
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float* __restrict__ part, int ks,
                                                            int inter, uint16_t* __restrict__ act) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  const int r = blockIdx.y;
  if (i >= inter) return;
  const size_t stride = static_cast<size_t>(gridDim.y) * 2 * inter;
  const float* row = part + static_cast<size_t>(r) * 2 * inter;
  const float g = round_bf(sum_splits(row + i, stride, ks));
  const float u = round_bf(sum_splits(row + inter + i, stride, ks));
  act[static_cast<size_t>(r) * inter + i] =
      static_cast<uint16_t>(f2bf(round_bf(g / (1.0f + expf(-g))) * u));
}

// SwiGLU over an f32 gate|up product with interleaved columns (column 2i =
// gate_i, 2i + 1 = up_i: the decode layout of the fused weight), four pairs a
// thread: act[r, i] = bf16(bf16(silu(bf16 g)) * bf16 u), the arithmetic of the
// decode step's fused epilogue. examples/qwen3_1_7b-tilelang/fast/kernels.py:210-257
// (gemv_silu's prologue) and :547-572 (silu_mul).
__global__ __launch_bounds__(kThreads) void swiglu_pairs_kernel(const float* __restrict__ gu, int ks, int64_t ld,
                                                                int64_t rows, int inter,
                                                                uint16_t* __restrict__ act) {
  const int per_row = inter / 4;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= rows * per_row) return;
  const int64_t r = e / per_row;
  const int i0 = static_cast<int>(e % per_row) * 4;
  float s[8];
  sum_splits8(gu + r * ld + 2 * i0, static_cast<size_t>(rows * ld), ks, s);   // split-K partials in split order
  const float g[4] = {s[0], s[2], s[4], s[6]}, u[4] = {s[1], s[3], s[5], s[7]};
  float y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float gb = round_bf(g[j]), ub = round_bf(u[j]);
    y[j] = round_bf(round_bf(gb / (1.0f + expf(-gb))) * ub);
  }
  *reinterpret_cast<uint2*>(act + r * inter + i0) = make_uint2(pack_bf(y[0], y[1]), pack_bf(y[2], y[3]));
}

// out[r, :] = table[ids[r], :], or bf16(table[ids[r], :] * scale) when `scaled`.
// 16 bytes a thread. An id outside [0, vocab) reads row 0 and sets err = 1.
// examples/qwen3_1_7b-tilelang/fast/kernels.py:579-588 (embed) and
// examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:72-76 (embed_scaled).
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint16_t* __restrict__ table,
                                                         const int64_t* __restrict__ ids,
                                                         int64_t vocab, int hidden, int scaled,
                                                         float scale, uint16_t* __restrict__ out,
                                                         int* err) {
  const int c = blockIdx.x * kThreads + threadIdx.x;  // 8-element chunk
  const int r = blockIdx.y;
  if (8 * c >= hidden) return;
  int64_t id = ids[r];
  if (id < 0 || id >= vocab) {
    if (c == 0) set_err(err, 1);
    id = 0;
  }
  uint4 v = ld16(table + id * hidden + 8 * c);
  if (scaled) {
    float f[8];
    unpack8(v, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = round_bf(f[i] * scale);
    v = pack8(f);
  }
  st16(out + static_cast<size_t>(r) * hidden + 8 * c, v);
}

}  // namespace

extern "C" {

int64_t tfa_lm_head_blocks(int64_t vocab) { return (vocab + kLmHeadRows - 1) / kLmHeadRows; }

int tfa_gemv(const void* x, const void* w, void* y, int64_t n, int64_t k, int out_f32,
             hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.N = (int)n;
  a.K = (int)k;
  TFA_TRY(check_gemv(a, "tfa_gemv"));
  TFA_TRY(check_vec(x, "x", "tfa_gemv"));
  if (!y) return fail(TFA_ERR_NULL, "tfa_gemv: null y");
  if (out_f32) {
    a.yf = static_cast<float*>(y);
    return dispatch_rows<PRO_PLAIN, EPI_F32>(a, stream, "gemv");
  }
  a.yb = static_cast<uint16_t*>(y);
  return dispatch_rows<PRO_PLAIN, EPI_BF16>(a, stream, "gemv");
}

int tfa_rmsnorm_gemv(const void* h, const void* gamma, float eps, const void* w, void* y,
                     int64_t n, int64_t k, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.gamma = static_cast<const uint16_t*>(gamma);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(w);
  a.N = (int)n;
  a.K = (int)k;
  a.yb = static_cast<uint16_t*>(y);
  TFA_TRY(check_gemv(a, "tfa_rmsnorm_gemv"));
  TFA_TRY(check_vec(h, "h", "tfa_rmsnorm_gemv"));
  TFA_TRY(check_vec(gamma, "gamma", "tfa_rmsnorm_gemv"));
  if (!y) return fail(TFA_ERR_NULL, "tfa_rmsnorm_gemv: null y");
  return dispatch_rows<PRO_NORM, EPI_BF16>(a, stream, "rmsnorm_gemv");
}

int tfa_rmsnorm_gemv_f32(const void* h, const void* gamma, float eps, const void* w, float* y,
                         int64_t n, int64_t k, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.gamma = static_cast<const uint16_t*>(gamma);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(w);
  a.N = (int)n;
  a.K = (int)k;
  a.yf = y;
  TFA_TRY(check_gemv(a, "tfa_rmsnorm_gemv_f32"));
  TFA_TRY(check_vec(h, "h", "tfa_rmsnorm_gemv_f32"));
  TFA_TRY(check_vec(gamma, "gamma", "tfa_rmsnorm_gemv_f32"));
  if (!y) return fail(TFA_ERR_NULL, "tfa_rmsnorm_gemv_f32: null y");
  return dispatch_rows<PRO_NORM, EPI_F32>(a, stream, "rmsnorm_gemv_f32");
}

int tfa_mla_prep_q_gemv(const float* part, int64_t q_lora, const void* gamma_q_a, const void* gamma_kv_a,
                        float eps, const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos,
                        void* latent_cache, void* rope_cache, int64_t cap, const void* w_q_b, float* q_part,
                        int64_t n, int* err, hipStream_t stream) {
  static const char* name = "tfa_mla_prep_q_gemv";
  GemvArgs a{};
  a.w = static_cast<const uint16_t*>(w_q_b);
  a.N = (int)n;
  a.K = (int)q_lora;
  TFA_TRY(check_gemv(a, name));
  if (q_lora > 4 * kThreads) return fail(TFA_ERR_SHAPE, "%s: q_lora %lld exceeds %d", name, (long long)q_lora, 4 * kThreads);
  TFA_TRY(check_vec(part, "part", name));
  TFA_TRY(check_vec(gamma_q_a, "gamma_q_a", name));
  if (!gamma_kv_a || !cos_t || !sin_t || !pos || !latent_cache || !rope_cache || !q_part)
    return fail(TFA_ERR_NULL, "%s: null argument", name);
  if (cap < 1 || rope_rows < 1) return fail(TFA_ERR_SHAPE, "%s: empty cache or rope table", name);
  a.xf = part;
  a.gamma = static_cast<const uint16_t*>(gamma_q_a);
  a.gkv = static_cast<const uint16_t*>(gamma_kv_a);
  a.eps = eps;
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.rope_rows = (int)rope_rows;
  a.pos = pos;
  a.lat_cache = static_cast<uint16_t*>(latent_cache);
  a.rope_cache = static_cast<uint16_t*>(rope_cache);
  a.cap = (int)cap;
  a.yf = q_part;
  a.err = err;
  // q_lora <= 1024 is one 16-byte chunk per lane; rows per block as dispatch_rows
  if (a.N <= 2560) return launch_gemv<1, 2, PRO_LORA, EPI_F32>(a, stream, "mla_prep_q_gemv");
  if (a.N < 16384) return launch_gemv<1, 4, PRO_LORA, EPI_F32>(a, stream, "mla_prep_q_gemv");
  return launch_gemv<1, 8, PRO_LORA, EPI_F32>(a, stream, "mla_prep_q_gemv");
}

int tfa_gemv_residual(const void* x, const void* w, const void* residual, const void* alpha,
                      void* y, int64_t n, int64_t k, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.res = static_cast<const uint16_t*>(residual);
  a.alpha = static_cast<const uint16_t*>(alpha);
  a.yb = static_cast<uint16_t*>(y);
  a.N = (int)n;
  a.K = (int)k;
  TFA_TRY(check_gemv(a, "tfa_gemv_residual"));
  TFA_TRY(check_vec(x, "x", "tfa_gemv_residual"));
  if (!residual || !y) return fail(TFA_ERR_NULL, "tfa_gemv_residual: null residual / y");
  if (alpha) return dispatch_rows<PRO_PLAIN, EPI_RESID_SCALED>(a, stream, "gemv_residual");
  return dispatch_rows<PRO_PLAIN, EPI_RESID>(a, stream, "gemv_residual");
}

int tfa_rmsnorm_gemv_swiglu(const void* h, const void* gamma, float eps, const void* w_gu,
                            void* act, int64_t inter, int64_t k, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.gamma = static_cast<const uint16_t*>(gamma);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(w_gu);
  a.N = (int)(2 * inter);
  a.K = (int)k;
  a.yb = static_cast<uint16_t*>(act);
  TFA_TRY(check_gemv(a, "tfa_rmsnorm_gemv_swiglu"));
  TFA_TRY(check_vec(h, "h", "tfa_rmsnorm_gemv_swiglu"));
  TFA_TRY(check_vec(gamma, "gamma", "tfa_rmsnorm_gemv_swiglu"));
  if (!act) return fail(TFA_ERR_NULL, "tfa_rmsnorm_gemv_swiglu: null act");
  return dispatch_rows<PRO_NORM, EPI_SWIGLU>(a, stream, "rmsnorm_gemv_swiglu");
}

int tfa_lm_head_argmax(const void* h, const void* gamma, float eps, const void* w, int64_t vocab,
                       int64_t k, float* logits, float* block_val, int* block_idx,
                       hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.gamma = static_cast<const uint16_t*>(gamma);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(w);
  a.N = (int)vocab;
  a.K = (int)k;
  a.yf = logits;
  a.bv = block_val;
  a.bi = block_idx;
  TFA_TRY(check_gemv(a, "tfa_lm_head_argmax"));
  TFA_TRY(check_vec(h, "h", "tfa_lm_head_argmax"));
  if (!logits || !block_val || !block_idx)
    return fail(TFA_ERR_NULL, "tfa_lm_head_argmax: null logits / block buffers");
  if (gamma) {
    TFA_TRY(check_vec(gamma, "gamma", "tfa_lm_head_argmax"));
    return dispatch_k<kLmHeadRows, PRO_NORM, EPI_ARGMAX>(a, stream, "lm_head_argmax");
  }
  return dispatch_k<kLmHeadRows, PRO_PLAIN, EPI_ARGMAX>(a, stream, "lm_head_argmax");
}

int tfa_sample_step(const float* block_val, const int* block_idx, int64_t nblocks, const int* inp,
                    const int* prompt_len, int64_t* ids, int* pos, int* sam, int64_t nsteps,
                    int* err, hipStream_t stream) {
  if (!block_val || !block_idx || !inp || !prompt_len || !ids || !pos || !sam)
    return fail(TFA_ERR_NULL, "tfa_sample_step: null pointer argument");
  if (nblocks <= 0 || nsteps <= 0) return fail(TFA_ERR_SHAPE, "tfa_sample_step: empty block list or step table");
  sample_kernel<<<1, kSampleThreads, 0, stream>>>(block_val, block_idx, (int)nblocks, inp, prompt_len,
                                            ids, pos, sam, (int)nsteps, err);
  return launched("sample_step");
}

int tfa_decode_qkv(const void* h, const void* table, const int64_t* ids, int64_t vocab,
                   void* h_copy, const void* gamma_in, float eps, const void* w_qkv,
                   int64_t hidden, int64_t n_qk, int64_t n_v, void* qk_out, const int* wr,
                   void* v_cache, int64_t cap, int* err, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.table = static_cast<const uint16_t*>(table);
  a.ids = ids;
  a.vocab = vocab;
  a.h_copy = static_cast<uint16_t*>(h_copy);
  a.gamma = static_cast<const uint16_t*>(gamma_in);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(w_qkv);
  a.K = (int)hidden;
  a.N = (int)(n_qk + n_v);
  a.n_qk = (int)n_qk;
  a.yb = static_cast<uint16_t*>(qk_out);
  a.wr = wr;
  a.cap = (int)cap;
  a.vc = static_cast<uint16_t*>(v_cache);
  a.err = err;
  TFA_TRY(check_gemv(a, "tfa_decode_qkv"));
  if (n_qk <= 0 || n_v <= 0) return fail(TFA_ERR_SHAPE, "tfa_decode_qkv: empty q|k or v rows");
  if (!gamma_in || !qk_out || !wr || !v_cache)
    return fail(TFA_ERR_NULL, "tfa_decode_qkv: null pointer argument");
  TFA_TRY(check_vec(gamma_in, "gamma_in", "tfa_decode_qkv"));
  if (cap <= 0) return fail(TFA_ERR_SHAPE, "tfa_decode_qkv: empty cache");
  if (table) {
    if (!ids || !h_copy) return fail(TFA_ERR_NULL, "tfa_decode_qkv: embed mode needs ids and h_copy");
    TFA_TRY(check_vec(table, "table", "tfa_decode_qkv"));
    TFA_TRY(check_vec(h_copy, "h_copy", "tfa_decode_qkv"));
    return dispatch_rows<PRO_EMBED_NORM, EPI_QKV>(a, stream, "decode_qkv");
  }
  TFA_TRY(check_vec(h, "h", "tfa_decode_qkv"));
  return dispatch_rows<PRO_NORM, EPI_QKV>(a, stream, "decode_qkv");
}

int tfa_rmsnorm_gemv_gate_up(const void* h, const void* gamma, float eps, const void* w_gate,
                             const void* w_up, void* act, int64_t inter, int64_t k,
                             hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.gamma = static_cast<const uint16_t*>(gamma);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(w_gate);
  a.w_odd = static_cast<const uint16_t*>(w_up);
  a.N = (int)(2 * inter);
  a.K = (int)k;
  a.yb = static_cast<uint16_t*>(act);
  TFA_TRY(check_gemv(a, "tfa_rmsnorm_gemv_gate_up"));
  TFA_TRY(check_vec(w_up, "w_up", "tfa_rmsnorm_gemv_gate_up"));
  TFA_TRY(check_vec(h, "h", "tfa_rmsnorm_gemv_gate_up"));
  TFA_TRY(check_vec(gamma, "gamma", "tfa_rmsnorm_gemv_gate_up"));
  if (!act) return fail(TFA_ERR_NULL, "tfa_rmsnorm_gemv_gate_up: null act");
  return dispatch_rows<PRO_NORM, EPI_SWIGLU>(a, stream, "rmsnorm_gemv_gate_up");
}

int tfa_lm_head_gemv(const void* h, const void* w, float divisor, void* logits, int64_t vocab,
                     int64_t k, hipStream_t stream) {
  GemvArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.w = static_cast<const uint16_t*>(w);
  a.in_div = divisor;
  a.N = (int)vocab;
  a.K = (int)k;
  a.yb = static_cast<uint16_t*>(logits);
  TFA_TRY(check_gemv(a, "tfa_lm_head_gemv"));
  TFA_TRY(check_vec(h, "h", "tfa_lm_head_gemv"));
  if (!logits) return fail(TFA_ERR_NULL, "tfa_lm_head_gemv: null logits");
  if (!(divisor != 0.f)) return fail(TFA_ERR_ARG, "tfa_lm_head_gemv: divisor must be nonzero");
  return dispatch_rows<PRO_PLAIN, EPI_BF16>(a, stream, "lm_head_gemv");
}

int tfa_silu_mul(const float* part, int64_t ks, int64_t inter, int64_t rows, void* act,
                 hipStream_t stream) {
  if (!part || !act) return fail(TFA_ERR_NULL, "tfa_silu_mul: null pointer argument");
  if (ks < 1 || ks > kMaxSplitsK) return fail(TFA_ERR_SHAPE, "tfa_silu_mul: ks %lld not in [1, %d]", (long long)ks, kMaxSplitsK);
  if (inter <= 0 || rows < 1 || rows > 65535) return fail(TFA_ERR_SHAPE, "tfa_silu_mul: bad shape");
  const dim3 grid((unsigned)((inter + kThreads - 1) / kThreads), (unsigned)rows);
  silu_mul_kernel<<<grid, kThreads, 0, stream>>>(part, (int)ks, (int)inter,
                                                  static_cast<uint16_t*>(act));
  return launched("silu_mul");
}

int tfa_swiglu_pairs(const float* gu, int64_t ld, int64_t rows, int64_t inter, void* act, hipStream_t stream) {
  return tfa_swiglu_pairs_split(gu, 1, ld, rows, inter, act, stream);
}

int tfa_swiglu_pairs_split(const float* gu, int64_t ks, int64_t ld, int64_t rows, int64_t inter, void* act,
                           hipStream_t stream) {
  if (!gu || !act) return fail(TFA_ERR_NULL, "tfa_swiglu_pairs: null pointer argument");
  if (ks < 1 || ks > kMaxSplitsK) return fail(TFA_ERR_SHAPE, "tfa_swiglu_pairs: ks %lld not in [1, %d]", (long long)ks, kMaxSplitsK);
  if (inter < 4 || inter % 4 || rows < 1 || ld < 2 * inter || ld % 4)
    return fail(TFA_ERR_SHAPE, "tfa_swiglu_pairs: inter %lld must be a positive multiple of 4, ld >= 2 inter "
                "and a multiple of 4", (long long)inter);
  if (!aligned16(gu) || (reinterpret_cast<uintptr_t>(act) & 7))
    return fail(TFA_ERR_ALIGN, "tfa_swiglu_pairs: gu must be 16-byte, act 8-byte aligned");
  const int64_t threads = rows * (inter / 4);
  if ((threads + kThreads - 1) / kThreads > INT32_MAX) return fail(TFA_ERR_SHAPE, "tfa_swiglu_pairs: too many rows");
  swiglu_pairs_kernel<<<(unsigned)((threads + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
      gu, (int)ks, ld, rows, (int)inter, static_cast<uint16_t*>(act));
  return launched("swiglu_pairs");
}

int tfa_embed(const void* table, const int64_t* ids, int64_t vocab, int64_t hidden, int64_t rows,
              int scaled, float scale, void* out, int* err, hipStream_t stream) {
  if (!table || !ids || !out) return fail(TFA_ERR_NULL, "tfa_embed: null pointer argument");
  if (hidden <= 0 || hidden % 8 != 0 || vocab <= 0 || rows < 1 || rows > 65535)
    return fail(TFA_ERR_SHAPE, "tfa_embed: hidden %lld must be a positive multiple of 8", (long long)hidden);
  if (!aligned16(table) || !aligned16(out)) return fail(TFA_ERR_ALIGN, "tfa_embed: table / out not 16-byte aligned");
  const dim3 grid((unsigned)((hidden / 8 + kThreads - 1) / kThreads), (unsigned)rows);
  embed_kernel<<<grid, kThreads, 0, stream>>>(static_cast<const uint16_t*>(table), ids, vocab,
                                               (int)hidden, scaled, scale,
                                               static_cast<uint16_t*>(out), err);
  return launched("embed");
}

}  // extern "C"
