// Decode (one token per sequence) kernels for weights stored [N, K] (out, in).
//
// gemv_rows: y[n] = sum_k x[k] W[n, k]. A 256-thread block owns R consecutive
// rows; its four waves split K into contiguous quarters, so each wave reads a
// contiguous 1 KB run of every row per load instruction (16 bytes a lane) and
// the block's partial dots meet in LDS in wave order (deterministic). The whole
// output of a row is produced by one block: no split-K partials leave the
// kernel. Weight loads are issued first; the input-vector prologue (a norm over
// the full hidden vector, recomputed by every block from a 4 KB row that sits
// in L2) runs while they are in flight.
//
// Prologues:   plain x | rmsnorm(h) | rmsnorm(embed[ids[0]])
// Epilogues:   f32 | bf16 | residual add | scaled residual add | SwiGLU pair |
//              logits + argmax + greedy sample step | q/k head norm + RoPE +
//              KV-cache write
// The last two finish work that needs a whole row group (a head, the
// vocabulary) in whichever block of the group arrives last.
//
// attn_decode: split-KV GQA attention of one query position against the
// cached positions 0..pos, one block per (split, kv head), the splits merged by
// log-sum-exp in the last block of each kv head.
//
// Reference kernels replaced: examples/qwen3_1_7b-tilelang/fast/kernels.py
// (gemv :123-145, gemv_attn_combine :154-207, gemv_silu :210-257, lm_head
// :260-321, qk_rope_cache :328-411, attn_partial :418-501, attn_combine
// :504-540, embed :579-588, sample_step :591-637) and the MiniCPM3 GEMVs
// examples/minicpm3_4b-cutedsl/kernels/cute_gemv.py:246-495.
#include <float.h>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kQkvRows = 8;      // rows per block of the fused qkv GEMV (divides head_dim)
constexpr int kLmHeadRows = 16;  // rows per block of the head (one argmax candidate each)

enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_EMBED_NORM = 2 };
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
  int N, K;
  // outputs
  float* yf;              // f32 out / logits
  uint16_t* yb;           // bf16 out
  const uint16_t* res;    // [N] residual
  const uint16_t* alpha;  // [1] bf16 residual scale (scaled residual)
  // argmax + sample
  float* bv;              // [gridDim.x] block maxima
  int* bi;                // [gridDim.x] their indices
  unsigned int* counter;  // [1] (argmax) / [HQ + HKV] (qkv)
  const int* inp;         // [nsteps] prompt ids
  const int* plen;        // [1] prompt length
  int64_t* ids_out;       // [1] next input id
  int* pos;               // [1] position (read by qkv, advanced by sample)
  int* sam;               // [nsteps] picks
  int nsteps;
  int* err;               // [1] device-side index error flag (may be null)
  // q/k norm + rope + cache write
  const uint16_t* gq;     // [D]
  const uint16_t* gk;     // [D]
  const uint16_t* cos_t;  // [MP, D]
  const uint16_t* sin_t;  // [MP, D]
  int mp;                 // rows of the rope tables
  const int* wr;          // [1] cache slot to write
  int cap;                // cache capacity (positions)
  uint16_t* kc;           // [cap, HKV*D]
  uint16_t* vc;           // [cap, HKV*D]
  uint16_t* q;            // [HQ*D]
  float* scratch;         // [(HQ+HKV)*D]
  int hq, hkv, hd;
  float eps_head;
};

TFA_DEV void set_err(int* err, int code) {
  if (err) atomicExch(err, code);
}

// (value, index) pair order for greedy argmax: larger value wins, equal values
// go to the lower index (torch.argmax), NaN never wins.
TFA_DEV bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int NCH, int R, int PRO, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_rows_kernel(const GemvArgs a) {
  __shared__ float red[kWaves][R];
  __shared__ float ssq[kWaves];
  __shared__ float hrow[256];
  __shared__ float rv_s[kThreads];
  __shared__ int ri_s[kThreads];
  __shared__ int flag;

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int row0 = blockIdx.x * R;
  const int K = a.K;
  const int kq = K / kWaves;   // elements in this wave's quarter
  const int nch = kq >> 3;     // 16-byte chunks in the quarter
  const int kbase = wid * kq;

  // 1. weights, first: they do not depend on the prologue
  uint4 w[R][NCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + j * kWave;
      if (row < a.N && c < nch)
        w[r][j] = ld16_stream(a.w + static_cast<size_t>(row) * K + kbase + 8 * c);
      else
        w[r][j] = make_uint4(0, 0, 0, 0);
    }
  }

  // 2. this wave's quarter of the input vector
  const uint16_t* src = a.x;
  if (PRO == PRO_EMBED_NORM) {
    int64_t id = a.ids[0];
    if (id < 0 || id >= a.vocab) {
      if (blockIdx.x == 0 && threadIdx.x == 0) set_err(a.err, 1);
      id = 0;
    }
    src = a.table + id * K;
  }
  float xf[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + j * kWave;
    if (c < nch) {
      const uint4 v = ld16(src + kbase + 8 * c);
      if (PRO == PRO_EMBED_NORM && blockIdx.x == 0) st16(a.h_copy + kbase + 8 * c, v);
      unpack8(v, xf[j]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xf[j][i] = 0.f;
    }
  }
  if (PRO != PRO_PLAIN) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += xf[j][i] * xf[j][i];
    ss = wave_sum(ss);
    if (lane == 0) ssq[wid] = ss;
    __syncthreads();
    const float tot = (ssq[0] + ssq[1]) + (ssq[2] + ssq[3]);
    const float rs = rsqrt_rn(tot / static_cast<float>(K) + a.eps);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + j * kWave;
      if (c < nch) {
        float g[8];
        unpack8(ld16(a.gamma + kbase + 8 * c), g);
#pragma unroll
        for (int i = 0; i < 8; ++i) xf[j][i] = round_bf(round_bf(xf[j][i] * rs) * g[i]);
      }
    }
  }

  // 3. dots
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
    acc[r] = wave_sum(s);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) red[wid][r] = acc[r];
  }
  __syncthreads();
  const int t = threadIdx.x;
  auto total = [&](int r) { return (red[0][r] + red[1][r]) + (red[2][r] + red[3][r]); };

  // 4. epilogues
  if (EPI == EPI_F32 || EPI == EPI_BF16 || EPI == EPI_RESID || EPI == EPI_RESID_SCALED) {
    if (t < R && row0 + t < a.N) {
      const int row = row0 + t;
      const float v = total(t);
      if (EPI == EPI_F32) a.yf[row] = v;
      if (EPI == EPI_BF16) a.yb[row] = static_cast<uint16_t>(f2bf(v));
      if (EPI == EPI_RESID) a.yb[row] = static_cast<uint16_t>(f2bf(bf2f(a.res[row]) + round_bf(v)));
      if (EPI == EPI_RESID_SCALED) {
        const float al = bf2f(a.alpha[0]);
        a.yb[row] = static_cast<uint16_t>(f2bf(bf2f(a.res[row]) + round_bf(round_bf(v) * al)));
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
    if (arrive_last(a.counter, gridDim.x, &flag)) {
      float bvv = -FLT_MAX;
      int bii = 0x7fffffff;
      for (int b = t; b < static_cast<int>(gridDim.x); b += kThreads) {
        const float v = a.bv[b];
        const int i = a.bi[b];
        if (better(v, i, bvv, bii)) { bvv = v; bii = i; }
      }
      rv_s[t] = bvv;
      ri_s[t] = bii;
      __syncthreads();
      for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (t < s && better(rv_s[t + s], ri_s[t + s], rv_s[t], ri_s[t])) {
          rv_s[t] = rv_s[t + s];
          ri_s[t] = ri_s[t + s];
        }
        __syncthreads();
      }
      if (t == 0 && a.pos != nullptr) {
        // the greedy sample step: record, feed the next prompt id or the pick, advance
        const int best = ri_s[0];
        const int p = a.pos[0];
        if (p < 0 || p >= a.nsteps) {
          set_err(a.err, 2);
        } else {
          a.sam[p] = best;
          const bool prompt = (p + 1 < a.plen[0]) && (p + 1 < a.nsteps);
          a.ids_out[0] = prompt ? static_cast<int64_t>(a.inp[p + 1]) : static_cast<int64_t>(best);
          a.pos[0] = p + 1;
        }
      }
    }
  }

  if (EPI == EPI_QKV) {
    const int D = a.hd;
    const int head = row0 / D;  // R divides D: a block lies inside one head
    const int nqk = a.hq + a.hkv;
    if (head >= nqk) {
      // value head: lands in the cache as it is
      if (t < R) {
        const int wslot = a.wr[0];
        if (wslot < 0 || wslot >= a.cap) {
          if (t == 0) set_err(a.err, 3);
        } else {
          const int vh = head - nqk;
          a.vc[static_cast<size_t>(wslot) * a.hkv * D + vh * D + (row0 % D) + t] =
              static_cast<uint16_t>(f2bf(total(t)));
        }
      }
    } else {
      if (t < R) a.scratch[row0 + t] = round_bf(total(t));
      if (arrive_last(&a.counter[head], D / R, &flag)) {
        // the head is complete: RMSNorm over D, rotate-half RoPE at pos
        const bool is_q = head < a.hq;
        const float x = t < D ? a.scratch[head * D + t] : 0.f;
        const float ss = block_sum(x * x, ssq);
        const float rs = rsqrt_rn(ss / static_cast<float>(D) + a.eps_head);
        const uint16_t* gam = is_q ? a.gq : a.gk;
        if (t < D) hrow[t] = round_bf(round_bf(x * rs) * bf2f(gam[t]));
        __syncthreads();
        const int p = a.pos[0];
        const int wslot = a.wr[0];
        const bool ok = p >= 0 && p < a.mp && (is_q || (wslot >= 0 && wslot < a.cap));
        if (!ok) {
          if (t == 0) set_err(a.err, 3);
        } else if (t < D) {
          const int h2 = D / 2;
          const float nv = hrow[t];
          const float half = t < h2 ? -hrow[t + h2] : hrow[t - h2];
          const float c = bf2f(a.cos_t[static_cast<size_t>(p) * D + t]);
          const float s = bf2f(a.sin_t[static_cast<size_t>(p) * D + t]);
          const uint16_t out = static_cast<uint16_t>(f2bf(__fadd_rn(__fmul_rn(nv, c), __fmul_rn(half, s))));
          if (is_q) a.q[head * D + t] = out;
          else a.kc[static_cast<size_t>(wslot) * a.hkv * D + (head - a.hq) * D + t] = out;
        }
      }
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

// ------------------------------------------------------------- attention
// Split-KV decode attention. Block (split s, kv head h) scores its G query
// heads against positions [s*SS, s*SS + SS) that are <= pos, normalises them
// against the split's own max (f32), lands the weights in bf16 and accumulates
// P.V in f32 -- the order of examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501.
// Lanes: slot = lane / 16 picks one of four positions, dc = lane % 16 one 8-wide
// slice of D = 128, so a wave reads four whole 256-byte key rows per load.
struct AttnArgs {
  const uint16_t* q;   // [HQ*D]
  const uint16_t* kc;  // [cap, HKV*D]
  const uint16_t* vc;  // [cap, HKV*D]
  const int* pos;      // [1] attend positions 0..pos
  float* op;           // [NS, HQ, D]
  float* mp;           // [NS, HQ]
  float* lp;           // [NS, HQ]
  unsigned int* counter;  // [HKV] (merge in-kernel) or null (partials only)
  uint16_t* out;       // [HQ*D] merged output (when counter is given)
  int* err;
  int hq, hkv, cap, ns;
  float scale;
};

template <int G, int NIT>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(const AttnArgs a) {
  constexpr int D = 128;
  constexpr int SS = 16 * NIT;
  __shared__ float sc[G][SS];
  __shared__ float obuf[kWaves][G][D];
  __shared__ float redm[kWaves];
  __shared__ int flag;

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int slot = lane >> 4;
  const int dc = lane & 15;
  const int s = blockIdx.x;
  const int kvh = blockIdx.y;
  const int t = threadIdx.x;
  const int KN = a.hkv * D;

  int p = a.pos[0];
  if (p < 0 || p >= a.cap) {
    if (s == 0 && kvh == 0 && t == 0) set_err(a.err, 4);
    p = p < 0 ? -1 : a.cap - 1;
  }
  const int n = p + 1;
  const int start = s * SS;

  if (start < n) {
    float qf[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) unpack8(ld16(a.q + (kvh * G + g) * D + 8 * dc), qf[g]);
    uint4 kv[NIT], vv[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int pi = start + it * 16 + wid * 4 + slot;
      const bool valid = pi < n;
      const size_t off = static_cast<size_t>(pi) * KN + kvh * D + 8 * dc;
      kv[it] = valid ? ld16_stream(a.kc + off) : make_uint4(0, 0, 0, 0);
      vv[it] = valid ? ld16_stream(a.vc + off) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      float kf[8];
      unpack8(kv[it], kf);
      const int li = it * 16 + wid * 4 + slot;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d = fmaf(qf[g][i], kf[i], d);
        d = group_sum<16>(d);
        if (dc == 0) sc[g][li] = (start + li < n) ? d * a.scale : -INFINITY;
      }
    }
    __syncthreads();
    // softmax over the split, one thread per position
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = t < SS ? sc[g][t] : -INFINITY;
      float mw = wave_max(v);
      if (lane == 0) redm[wid] = mw;
      __syncthreads();
      m[g] = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
      __syncthreads();
      const float e = (t < SS && start + t < n) ? expf(v - m[g]) : 0.f;
      l[g] = block_sum(e, redm);
      if (t < SS) sc[g][t] = round_bf(e);  // bf16 weights into the value product
    }
    __syncthreads();
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      float vf[8];
      unpack8(vv[it], vf);
      const int li = it * 16 + wid * 4 + slot;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pw = sc[g][li];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = fmaf(pw, vf[i], o[g][i]);
      }
    }
    // reduce the four position slots of each wave, then the four waves
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = o[g][i];
        v += __shfl_xor(v, 16, kWave);
        v += __shfl_xor(v, 32, kWave);
        o[g][i] = v;
      }
    if (slot == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) obuf[wid][g][8 * dc + i] = o[g][i];
    }
    __syncthreads();
    for (int e = t; e < G * D; e += kThreads) {
      const int g = e / D, d = e % D;
      const float v = (obuf[0][g][d] + obuf[1][g][d]) + (obuf[2][g][d] + obuf[3][g][d]);
      const int h = kvh * G + g;
      a.op[(static_cast<size_t>(s) * a.hq + h) * D + d] = v;
      if (d == 0) {
        a.mp[s * a.hq + h] = m[g];
        a.lp[s * a.hq + h] = l[g];
      }
    }
  } else if (a.counter == nullptr) {
    // partials-only form: a split past the context is neutral
    for (int e = t; e < G * D; e += kThreads) {
      const int g = e / D, d = e % D;
      const int h = kvh * G + g;
      a.op[(static_cast<size_t>(s) * a.hq + h) * D + d] = 0.f;
      if (d == 0) {
        a.mp[s * a.hq + h] = -1.0e30f;
        a.lp[s * a.hq + h] = 0.f;
      }
    }
  }

  if (a.counter != nullptr && arrive_last(&a.counter[kvh], a.ns, &flag)) {
    const int nact = (n + SS - 1) / SS;
    for (int e = t; e < G * D; e += kThreads) {
      const int g = e / D, d = e % D;
      const int h = kvh * G + g;
      float mx = -INFINITY;
      for (int j = 0; j < nact; ++j) mx = fmaxf(mx, a.mp[j * a.hq + h]);
      float den = 0.f, num = 0.f;
      for (int j = 0; j < nact; ++j) {
        const float ex = expf(a.mp[j * a.hq + h] - mx);
        den = fmaf(a.lp[j * a.hq + h], ex, den);
        num = fmaf(a.op[(static_cast<size_t>(j) * a.hq + h) * D + d], ex, num);
      }
      a.out[h * D + d] = static_cast<uint16_t>(f2bf(num / den));
    }
  }
}

template <int G>
int launch_attn_g(const AttnArgs& a, int ss, hipStream_t st) {
  const dim3 grid(a.ns, a.hkv);
  switch (ss) {
    case 64: attn_decode_kernel<G, 4><<<grid, kThreads, 0, st>>>(a); break;
    case 128: attn_decode_kernel<G, 8><<<grid, kThreads, 0, st>>>(a); break;
    case 256: attn_decode_kernel<G, 16><<<grid, kThreads, 0, st>>>(a); break;
    default: return fail(TFA_ERR_SHAPE, "attn_decode: split %d not in {64, 128, 256}", ss);
  }
  return launched("attn_decode");
}

// Merge of split partials into bf16 head-major output (no GEMV folded in).
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* op, const float* mp,
                                                           const float* lp, uint16_t* out,
                                                           int ns, int hq, int D) {
  const int h = blockIdx.x;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float mx = -1.0e30f;
    for (int s = 0; s < ns; ++s) mx = fmaxf(mx, mp[s * hq + h]);
    float den = 0.f, num = 0.f;
    for (int s = 0; s < ns; ++s) {
      const float e = expf(mp[s * hq + h] - mx);
      den = fmaf(lp[s * hq + h], e, den);
      num = fmaf(op[(static_cast<size_t>(s) * hq + h) * D + d], e, num);
    }
    out[h * D + d] = static_cast<uint16_t>(f2bf(num / den));
  }
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
    return n >= 4096 ? dispatch_k<8, PRO_PLAIN, EPI_F32>(a, stream, "gemv")
                     : dispatch_k<4, PRO_PLAIN, EPI_F32>(a, stream, "gemv");
  }
  a.yb = static_cast<uint16_t*>(y);
  return n >= 4096 ? dispatch_k<8, PRO_PLAIN, EPI_BF16>(a, stream, "gemv")
                   : dispatch_k<4, PRO_PLAIN, EPI_BF16>(a, stream, "gemv");
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
  return n >= 4096 ? dispatch_k<8, PRO_NORM, EPI_BF16>(a, stream, "rmsnorm_gemv")
                   : dispatch_k<4, PRO_NORM, EPI_BF16>(a, stream, "rmsnorm_gemv");
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
  if (alpha) return dispatch_k<4, PRO_PLAIN, EPI_RESID_SCALED>(a, stream, "gemv_residual");
  return dispatch_k<4, PRO_PLAIN, EPI_RESID>(a, stream, "gemv_residual");
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
  return dispatch_k<8, PRO_NORM, EPI_SWIGLU>(a, stream, "rmsnorm_gemv_swiglu");
}

int tfa_lm_head_sample(const void* h, const void* gamma, float eps, const void* w, int64_t vocab,
                       int64_t k, float* logits, float* block_val, int* block_idx,
                       unsigned int* counter, const int* inp, const int* prompt_len,
                       int64_t* ids, int* pos, int* sam, int64_t nsteps, int* err,
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
  a.counter = counter;
  a.inp = inp;
  a.plen = prompt_len;
  a.ids_out = ids;
  a.pos = pos;
  a.sam = sam;
  a.nsteps = (int)nsteps;
  a.err = err;
  TFA_TRY(check_gemv(a, "tfa_lm_head_sample"));
  TFA_TRY(check_vec(h, "h", "tfa_lm_head_sample"));
  if (!logits || !block_val || !block_idx || !counter)
    return fail(TFA_ERR_NULL, "tfa_lm_head_sample: null logits / block buffers / counter");
  if (pos && (!inp || !prompt_len || !ids || !sam))
    return fail(TFA_ERR_NULL, "tfa_lm_head_sample: sampling needs inp, prompt_len, ids, sam");
  const int PRO = gamma ? PRO_NORM : PRO_PLAIN;
  if (PRO == PRO_NORM) {
    TFA_TRY(check_vec(gamma, "gamma", "tfa_lm_head_sample"));
    return dispatch_k<kLmHeadRows, PRO_NORM, EPI_ARGMAX>(a, stream, "lm_head_sample");
  }
  return dispatch_k<kLmHeadRows, PRO_PLAIN, EPI_ARGMAX>(a, stream, "lm_head_sample");
}

int tfa_decode_qkv(const void* h, const void* table, const int64_t* ids, int64_t vocab,
                   void* h_copy, const void* gamma_in, float eps, const void* w_qkv,
                   int64_t hidden, int64_t hq, int64_t hkv, int64_t head_dim,
                   const void* gamma_q, const void* gamma_k, float eps_head, const void* cos_t,
                   const void* sin_t, int64_t rope_rows, const int* pos, const int* wr,
                   void* k_cache, void* v_cache, int64_t cap, void* q, float* scratch,
                   unsigned int* counters, int* err, hipStream_t stream) {
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
  a.N = (int)((hq + 2 * hkv) * head_dim);
  a.gq = static_cast<const uint16_t*>(gamma_q);
  a.gk = static_cast<const uint16_t*>(gamma_k);
  a.eps_head = eps_head;
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.mp = (int)rope_rows;
  a.pos = const_cast<int*>(pos);
  a.wr = wr;
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.cap = (int)cap;
  a.q = static_cast<uint16_t*>(q);
  a.scratch = scratch;
  a.counter = counters;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.hd = (int)head_dim;
  a.err = err;
  TFA_TRY(check_gemv(a, "tfa_decode_qkv"));
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(TFA_ERR_SHAPE, "tfa_decode_qkv: head_dim %lld not in {64, 128, 256}", (long long)head_dim);
  if (!gamma_in || !gamma_q || !gamma_k || !cos_t || !sin_t || !pos || !wr || !k_cache ||
      !v_cache || !q || !scratch || !counters)
    return fail(TFA_ERR_NULL, "tfa_decode_qkv: null pointer argument");
  if (cap <= 0 || rope_rows <= 0) return fail(TFA_ERR_SHAPE, "tfa_decode_qkv: empty cache or rope table");
  if (table) {
    if (!ids || !h_copy) return fail(TFA_ERR_NULL, "tfa_decode_qkv: embed mode needs ids and h_copy");
    TFA_TRY(check_vec(table, "table", "tfa_decode_qkv"));
    return dispatch_k<kQkvRows, PRO_EMBED_NORM, EPI_QKV>(a, stream, "decode_qkv");
  }
  TFA_TRY(check_vec(h, "h", "tfa_decode_qkv"));
  return dispatch_k<kQkvRows, PRO_NORM, EPI_QKV>(a, stream, "decode_qkv");
}

int tfa_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* pos,
                         int64_t hq, int64_t hkv, int64_t head_dim, int64_t cap, int64_t split,
                         float scale, float* op, float* mp, float* lp, unsigned int* counters,
                         void* out, int* err, hipStream_t stream) {
  if (!q || !k_cache || !v_cache || !pos || !op || !mp || !lp)
    return fail(TFA_ERR_NULL, "tfa_decode_attention: null pointer argument");
  if (counters && !out) return fail(TFA_ERR_NULL, "tfa_decode_attention: merge needs out");
  if (head_dim != 128) return fail(TFA_ERR_SHAPE, "tfa_decode_attention: head_dim %lld, only 128 supported", (long long)head_dim);
  if (hkv <= 0 || hq % hkv != 0) return fail(TFA_ERR_SHAPE, "tfa_decode_attention: hq %lld not a multiple of hkv %lld", (long long)hq, (long long)hkv);
  if (split <= 0 || cap <= 0 || cap % split != 0)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention: cap %lld not a positive multiple of split %lld", (long long)cap, (long long)split);
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(TFA_ERR_ALIGN, "tfa_decode_attention: q / caches not 16-byte aligned");
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.pos = pos;
  a.op = op;
  a.mp = mp;
  a.lp = lp;
  a.counter = counters;
  a.out = static_cast<uint16_t*>(out);
  a.err = err;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.cap = (int)cap;
  a.ns = (int)(cap / split);
  a.scale = scale;
  switch (hq / hkv) {
    case 1: return launch_attn_g<1>(a, (int)split, stream);
    case 2: return launch_attn_g<2>(a, (int)split, stream);
    case 4: return launch_attn_g<4>(a, (int)split, stream);
    case 8: return launch_attn_g<8>(a, (int)split, stream);
    default: return fail(TFA_ERR_SHAPE, "tfa_decode_attention: group %lld not in {1,2,4,8}", (long long)(hq / hkv));
  }
}

int tfa_attn_combine(const float* op, const float* mp, const float* lp, void* out, int64_t splits,
                     int64_t hq, int64_t head_dim, hipStream_t stream) {
  if (!op || !mp || !lp || !out) return fail(TFA_ERR_NULL, "tfa_attn_combine: null pointer argument");
  if (splits <= 0 || hq <= 0 || head_dim <= 0) return fail(TFA_ERR_SHAPE, "tfa_attn_combine: empty shape");
  attn_combine_kernel<<<(int)hq, 128, 0, stream>>>(op, mp, lp, static_cast<uint16_t*>(out),
                                                   (int)splits, (int)hq, (int)head_dim);
  return launched("attn_combine");
}

}  // extern "C"
