// Batched decode (up to 32 sequences, one token each): every projection is a
// skinny GEMM Y[M, N] = X[M, K] . W[N, K]^T with M <= 32 on bf16 MFMA.
//
// skinny_gemm: a 256-thread block owns 32 weight rows (two 16-wide MFMA column
// tiles) against all 32 token rows (two 16-high row tiles): four
// v_mfma_f32_16x16x32_bf16 per 32-wide k-step. K is split over the block's
// four waves (and optionally over `ks` blocks, each writing f32 partials that
// the consumer reduces, so the narrow 2048-row projections still fill every
// CU). The block walks its K range in steps of four 64-element chunks, one per
// wave (512 contiguous bytes of every row per step): the chunk's 32 weight
// rows and 32 token rows are loaded coalesced -- eight lanes per 128-byte row
// run, weights non-temporal -- into a wave-private LDS tile whose 144-byte row
// pitch makes the MFMA operand reads (16 rows, same column) bank-conflict
// free; the next chunk's loads are in flight while this chunk's MFMAs run. (A
// direct register load in MFMA layout would touch 32 rows per instruction, 16
// bytes each, and the lines are evicted before the next step uses them.)
// Lane layout of v_mfma_f32_16x16x32_bf16 (checked on the device):
//   A[i = l%16][k = 8*(l/16) + j], B[k = 8*(l/16) + j][n = l%16],
//   C[i = 4*(l/16) + r][n = l%16], j < 8, r < 4.
//
// Epilogues (each wave finishes one of the block's four 16x16 tiles): f32
// split-K partials | SwiGLU over interleaved gate/up rows | per token the best
// (value, lowest index) of every 16-row group, optionally with the f32 logits.
//
// rows_norm: per token row, either gather an embedding row or add the reduced
// split-K partials to the residual stream, then RMSNorm (mode 0) -- the
// producer-side norm that feeds the next GEMM.
//
// batch_sample: the greedy step for every sequence.
//
// Reference kernels replaced (batched form): examples/qwen3_1_7b-tilelang/fast/kernels.py
// gemv :123-145, gemv_silu :210-257, lm_head :260-321, resid_rms_norm :82-116,
// embed :579-588, sample_step :591-637.
#include <float.h>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxTokens = 32;
constexpr int kGroupRows = 16;   // argmax winners are kept per 16 weight rows

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { SK_PARTIAL = 0, SK_SWIGLU = 1, SK_ARGMAX = 2, SK_ARGMAX_BF16 = 3, SK_RESID_SSQ = 4 };

struct SkinnyArgs {
  const uint16_t* x;  // [M, K]
  const uint16_t* w;  // [N, K]
  int M, N, K, ks;
  float* part;        // [ks, M, N]
  uint16_t* act;      // [M, N/2]
  float* logits;      // [M, N] or null
  float* bv;          // [M, ngroups]
  int* bi;            // [M, ngroups]
  int ngroups;        // 16-row groups of N
  // residual epilogue: h_out[m, n] = bf16(res[m, n] + bf16(y)), and per block b
  // the token's sum of squares of its rows of h_out in ssq[b, m]
  const uint16_t* res;
  uint16_t* h_out;
  float* ssq;
  // norm prologue: x is the residual stream h; the token rows are staged as
  // bf16(bf16(h * r_m) * gamma), r_m = 1 / sqrt(sum_b ssq_in[b, m] / K + eps)
  const float* ssq_in;
  int nssq;
  const uint16_t* gamma;
  float eps;
};

TFA_DEV bf16x8 as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

TFA_DEV bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

constexpr int kChunk = 64;            // K elements per wave per pipeline step
constexpr int kLdsRow = kChunk + 8;   // padded LDS row (144 bytes): conflict-free 16-row reads

// Wave-private LDS staging, ordered by the wave's own in-order LDS pipeline: a
// compiler-level wave barrier keeps each chunk's stores, the other lanes' reads
// of them and the next chunk's stores in program order.
TFA_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int TR>
struct SkinnyStage {
  uint16_t w[TR][kLdsRow];            // the chunk's weight rows
  uint16_t x[kMaxTokens][kLdsRow];    // the chunk's token rows
};

// TR weight rows per block (32 or 48: TR / 16 MFMA column tiles) against the
// 32 token rows (two row tiles).
template <int EPI, int P, int TR, int W, bool NORM = false>
__global__ __launch_bounds__(W * kWave) void skinny_gemm_kernel(const SkinnyArgs a) {
  constexpr int RT = TR / 16;       // weight-row tiles
  constexpr int NT = 2 * RT;        // output tiles (token half, row tile)
  constexpr int WL = TR / 8;        // weight-row loads per lane per chunk
  static_assert(sizeof(SkinnyStage<TR>) >= NT * kWave * sizeof(float) * 4, "partials reuse the staging tile");
  static_assert(EPI != SK_RESID_SSQ || NT <= W, "the residual epilogue finishes one tile per wave");
  __shared__ SkinnyStage<TR> stage[W];   // reused for the block's partial sums
  __shared__ float rn[NORM ? kMaxTokens : 1];                       // the tokens' norm scales
  __shared__ float sq[NORM ? 8 : RT][kMaxTokens];                   // norm / ssq partials

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int grp = lane >> 4;
  const int r16 = lane & 15;
  const int n0 = blockIdx.x * TR;
  const int K = a.K;
  // the block's K range is walked in steps of W chunks, wave w taking chunk w
  // of each step: the block reads 128 W contiguous bytes of each row at a time
  const int kb = K / a.ks;                  // this block's K range
  const int nchunks = kb / (W * kChunk);   // chunks per wave
  const int kw0 = blockIdx.y * kb + wid * kChunk;
  constexpr int kStride = W * kChunk;  // K elements between a wave's chunks
  SkinnyStage<TR>& st = stage[wid];

  // coalesced staging: load i covers rows 8i .. 8i+7, eight lanes per 128-byte
  // row run. Weight rows past N and token rows past M re-read the last valid row
  // (in bounds, finite); the results they produce are never stored. Loads are
  // unconditional so the compiler can count them and wait only for the oldest.
  const int srow = lane >> 3;               // 0..7
  const int scol = (lane & 7) * 8;          // element offset in the chunk
  // Norm prologue, first of all (its loads complete first): thread t sums
  // ssq_in[b, t % 32] over b = 8 (t / 32) .. + 7 in order, the eight groups meet
  // in LDS in order, and r_m lands in rn[m] before the first chunk is staged.
  // (the first 256 threads: 8 groups of 8 of the at most 64 partial rows)
  float nsum = 0.f;
  const bool nthread = threadIdx.x < 8 * kMaxTokens;
  if constexpr (NORM) {
    const int m = threadIdx.x % kMaxTokens, g8 = min(static_cast<int>(threadIdx.x) / kMaxTokens, 7);
    float v8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int b = 8 * g8 + j;
      v8[j] = (nthread && b < a.nssq && m < a.M)
                  ? a.ssq_in[static_cast<size_t>(min(b, a.nssq - 1)) * a.M + min(m, a.M - 1)] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) nsum += v8[j];
  }
  // residual epilogue: this lane's residual values, loaded with the first loads
  uint32_t res_pre[4] = {0u, 0u, 0u, 0u};
  if constexpr (EPI == SK_RESID_SSQ) {
    if (wid < NT) {
      const int th = wid / RT, rh = wid % RT;
      const int n = min(n0 + 16 * rh + r16, a.N - 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) res_pre[r] = a.res[static_cast<size_t>(min(16 * th + 4 * grp + r, a.M - 1)) * a.N + n];
    }
  }
  const uint16_t* wp[WL];
  const uint16_t* xp[4];
#pragma unroll
  for (int i = 0; i < WL; ++i) {
    const int row = min(n0 + 8 * i + srow, a.N - 1);
    wp[i] = a.w + static_cast<size_t>(row) * K + kw0 + scol;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tok = min(8 * i + srow, a.M - 1);
    xp[i] = a.x + static_cast<size_t>(tok) * K + kw0 + scol;
  }
  // ring of P chunks in registers: chunk g*P + p lives in slot p (nchunks % P == 0)
  const uint16_t* gp = NORM ? a.gamma + kw0 + scol : nullptr;
  uint4 rw[P][WL], rx[P][4], rg[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
#pragma unroll
    for (int i = 0; i < WL; ++i) rw[p][i] = ld16_stream(wp[i] + p * kStride);
#pragma unroll
    for (int i = 0; i < 4; ++i) rx[p][i] = ld16(xp[i] + p * kStride);
    if constexpr (NORM) rg[p] = ld16(gp + p * kStride);
    __builtin_amdgcn_sched_barrier(0);   // issue the slots in order: slot p is waited for alone
  }
  float rtok[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (NORM) {
    if (nthread) sq[threadIdx.x / kMaxTokens][threadIdx.x % kMaxTokens] = nsum;
    __syncthreads();
    if (threadIdx.x < kMaxTokens) {
      float ss = 0.f;
#pragma unroll
      for (int g8 = 0; g8 < 8; ++g8) ss += sq[g8][threadIdx.x];
      rn[threadIdx.x] = rsqrt_rn(ss / static_cast<float>(K) + a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) rtok[i] = rn[8 * i + srow];
  }
  // a token chunk as staged: the residual stream normalised (norm prologue)
  auto token_chunk = [&](uint4 v, int i, uint4 g) __attribute__((always_inline)) {
    if constexpr (!NORM) return v;
    float f[8], gg[8];
    unpack8(v, f);
    unpack8(g, gg);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = round_bf(round_bf(f[e] * rtok[i]) * gg[e]);
    return pack8(f);
  };

  f32x4 c[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) c[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ngroups = nchunks / P;
  for (int g = 0; g < ngroups; ++g) {
    const bool refill = g + 1 < ngroups;   // wave-uniform
#pragma unroll
    for (int p = 0; p < P; ++p) {
      wave_lds_sync();   // the previous chunk's operand reads are issued before these stores
#pragma unroll
      for (int i = 0; i < WL; ++i) *reinterpret_cast<uint4*>(&st.w[8 * i + srow][scol]) = rw[p][i];
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&st.x[8 * i + srow][scol]) = token_chunk(rx[p][i], i, rg[p]);
      if (refill) {   // P chunks stay in flight during the MFMAs
        const int off = ((g + 1) * P + p) * kStride;
#pragma unroll
        for (int i = 0; i < WL; ++i) rw[p][i] = ld16_stream(wp[i] + off);
#pragma unroll
        for (int i = 0; i < 4; ++i) rx[p][i] = ld16(xp[i] + off);
        if constexpr (NORM) rg[p] = ld16(gp + off);
      }
      wave_lds_sync();
#pragma unroll
      for (int kk = 0; kk < kChunk / 32; ++kk) {
        const int col = kk * 32 + 8 * grp;
        uint4 wt[RT];
#pragma unroll
        for (int rh = 0; rh < RT; ++rh) wt[rh] = *reinterpret_cast<const uint4*>(&st.w[16 * rh + r16][col]);
        const uint4 xa = *reinterpret_cast<const uint4*>(&st.x[r16][col]);
        const uint4 xb = *reinterpret_cast<const uint4*>(&st.x[16 + r16][col]);
        // tile (token half th, row tile rh) = th * RT + rh: A = tokens, B = weight rows
#pragma unroll
        for (int rh = 0; rh < RT; ++rh) {
          c[rh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xa), as_bf8(wt[rh]), c[rh], 0, 0, 0);
          c[RT + rh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xb), as_bf8(wt[rh]), c[RT + rh], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();   // every wave is done with its staging tile
  f32x4 (*cbuf)[kWave] = reinterpret_cast<f32x4 (*)[kWave]>(&stage[wid]);
#pragma unroll
  for (int i = 0; i < NT; ++i) cbuf[i][lane] = c[i];
  __syncthreads();
  // wave w finishes tiles ti = w, w + 4, ...: lane (grp, r16) holds tokens
  // 16*th + 4*grp + r (r < 4) against weight row n0 + 16*rh + r16
  for (int ti = wid; ti < NT; ti += W) {
    const int th = ti / RT, rh = ti % RT;
    // pairwise over the waves' K ranges: ((0 + 1) + (2 + 3)) [+ ((4 + 5) + (6 + 7))]
    auto part = [&](int w) { return reinterpret_cast<const f32x4*>(&stage[w])[ti * kWave + lane]; };
    f32x4 s = (part(0) + part(1)) + (part(2) + part(3));
    if (W == 8) s += (part(4) + part(5)) + (part(6) + part(7));
    const int n = n0 + 16 * rh + r16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * th + 4 * grp + r;
      float val = s[r];
      if (EPI == SK_PARTIAL) {
        if (m < a.M && n < a.N) a.part[(static_cast<size_t>(blockIdx.y) * a.M + m) * a.N + n] = val;
      }
      if (EPI == SK_RESID_SSQ) {
        // h1 = bf16(h + bf16(y)); the tile's 16 rows of h1^2 summed per token
        const float h1 = round_bf(__uint_as_float(res_pre[r] << 16) + round_bf(val));
        const bool in = m < a.M && n < a.N;
        if (in) a.h_out[static_cast<size_t>(m) * a.N + n] = static_cast<uint16_t>(f2bf(h1));
        const float rs = row16_sum(in ? h1 * h1 : 0.f);
        if (r16 == 0) sq[rh][m] = rs;
      }
      if (EPI == SK_SWIGLU) {
        // rows (2i, 2i+1) = (gate_i, up_i) sit in lanes r16 and r16 ^ 1
        const float other = xor_lane<1>(val, r16);
        if ((r16 & 1) == 0 && m < a.M && n + 1 < a.N) {
          const float g = round_bf(val), u = round_bf(other);
          const float act = round_bf(round_bf(g / (1.0f + expf(-g))) * u);
          a.act[static_cast<size_t>(m) * (a.N / 2) + n / 2] = static_cast<uint16_t>(f2bf(act));
        }
      }
      if (EPI == SK_ARGMAX || EPI == SK_ARGMAX_BF16) {
        if (EPI == SK_ARGMAX_BF16) val = round_bf(val);   // bf16 logits: ties as the landed values have them
        if (a.logits && m < a.M && n < a.N) a.logits[static_cast<size_t>(m) * a.N + n] = val;
        // per token: best of the tile's 16 rows (lowest index on ties)
        float bvv = n < a.N ? val : -FLT_MAX;
        int bii = n < a.N ? n : 0x7fffffff;
        auto pick = [&](auto mc) __attribute__((always_inline)) {
          constexpr int M = decltype(mc)::value;
          const float ov = xor_lane<M>(bvv, r16);
          const int oi = xor_lane<M>(bii, r16);
          if (better(ov, oi, bvv, bii)) { bvv = ov; bii = oi; }
        };
        pick(std::integral_constant<int, 1>{});
        pick(std::integral_constant<int, 2>{});
        pick(std::integral_constant<int, 4>{});
        pick(std::integral_constant<int, 8>{});
        const int grp16 = n0 / kGroupRows + rh;   // this tile's 16-row group
        if (r16 == 0 && m < a.M && grp16 < a.ngroups) {
          a.bv[static_cast<size_t>(m) * a.ngroups + grp16] = bvv;
          a.bi[static_cast<size_t>(m) * a.ngroups + grp16] = bii;
        }
      }
    }
  }
  if constexpr (EPI == SK_RESID_SSQ) {   // the block's rows summed per token, row tiles in order
    __syncthreads();
    if (threadIdx.x < a.M) {
      float tot = 0.f;
#pragma unroll
      for (int rh = 0; rh < RT; ++rh) tot += sq[rh][threadIdx.x];
      a.ssq[static_cast<size_t>(blockIdx.x) * a.M + threadIdx.x] = tot;
    }
  }
}

// Register ring depth: two chunks in flight per wave when the wave's chunk count
// allows it (deeper rings cost occupancy and measured no faster).
int skinny_depth(int nchunks) { return nchunks % 2 == 0 ? 2 : 1; }

// Block height: 32 weight rows, or 48 when that fills the device in fewer
// rounds of one block per CU (e.g. 12288 rows: 384 blocks of 32 take two
// rounds on 256 CUs, 256 blocks of 48 take one of 1.5x the work).
int skinny_cus() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

template <int EPI, int TR, int W, bool NORM = false>
void launch_trw(const SkinnyArgs& a, hipStream_t st) {
  const dim3 grid((a.N + TR - 1) / TR, a.ks);
  if (skinny_depth(a.K / a.ks / W / kChunk) == 2)
    skinny_gemm_kernel<EPI, 2, TR, W, NORM><<<grid, W * kWave, 0, st>>>(a);
  else
    skinny_gemm_kernel<EPI, 1, TR, W, NORM><<<grid, W * kWave, 0, st>>>(a);
}

// Eight waves per block (two per SIMD) when the block's K range splits into
// 512-element steps: twice the loads in flight per CU of the four-wave form.
template <int EPI, int TR, bool NORM = false>
void launch_tr(const SkinnyArgs& a, hipStream_t st) {
  if ((a.K / a.ks) % (8 * kChunk) == 0)
    launch_trw<EPI, TR, 8, NORM>(a, st);
  else
    launch_trw<EPI, TR, 4, NORM>(a, st);
}

template <int EPI, bool NORM = false>
int launch_skinny(const SkinnyArgs& a, hipStream_t st, const char* name) {
  const int64_t cus = skinny_cus();
  auto cost = [&](int64_t tr) {   // rounds of resident blocks x rows per block
    const int64_t blocks = (a.N + tr - 1) / tr * a.ks;
    return (blocks + cus - 1) / cus * tr;
  };
  if constexpr (EPI == SK_RESID_SSQ)
    launch_tr<EPI, 32>(a, st);   // the residual epilogue's sums are per 32 rows
  else if (cost(48) < cost(32))
    launch_tr<EPI, 48, NORM>(a, st);
  else
    launch_tr<EPI, 32, NORM>(a, st);
  return launched(name);
}

// ---------------------------------------------------------------- rows_norm
// Per token row m (one 256-thread block; each thread owns 8-element chunks):
// h = table[ids[m]] (embed mode) or h = bf16(h_in[m] + bf16(sum_s part[s, m, :]))
// (residual mode), or with SCALED h = bf16(h_in[m] + bf16(bf16(sum_s part) * alpha))
// (MiniCPM3's scale_depth residual); h_out[m] = h;
// xn[m] = bf16(bf16(h * rsqrt(mean h^2 + eps)) * gamma).
// Every load of the row -- the residual or embedding row, the norm scale and
// MAXKS partial rows per chunk (clamped to the last of the ks) -- is issued,
// unconditionally at clamped addresses, before any of them is read: one memory
// round trip (two in embed mode, whose row address needs the id).
constexpr int kRowChunks = 2;   // 8-element chunks per thread: hidden <= 256 * 8 * 2
enum { RN_EMBED = 0, RN_RESID = 1, RN_RESID_SCALED = 2 };
template <int MODE, int MAXKS, int CH>
__global__ __launch_bounds__(kThreads) void rows_norm_kernel(
    const uint16_t* __restrict__ table, const int64_t* __restrict__ ids, int64_t vocab,
    const uint16_t* h_in, const float* __restrict__ part, int ks, uint16_t* h_out,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ xn, int M, int H, float eps,
    int* err, float alpha) {
  __shared__ float red[kWaves];
  const int m = blockIdx.x;
  const int t = threadIdx.x;
  const int nch = H / 8;
  const uint16_t* src;
  if constexpr (MODE == RN_EMBED) {
    int64_t id = ids[m];
    if (id < 0 || id >= vocab) {
      if (t == 0 && err) atomicExch(err, 1);
      id = 0;
    }
    src = table + id * H;
  } else {
    src = h_in + static_cast<size_t>(m) * H;
  }
  constexpr int KS = MODE == RN_EMBED ? 1 : MAXKS;
  uint4 hv[CH], gq[CH];
  float4 pv[CH][KS][2];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = min(t + c * kThreads, nch - 1);
    hv[c] = ld16(src + 8 * ch);
    gq[c] = ld16(gamma + 8 * ch);
    if constexpr (MODE != RN_EMBED) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const float4* q = reinterpret_cast<const float4*>(
            part + (static_cast<size_t>(min(s, ks - 1)) * M + m) * H + 8 * ch);
        pv[c][s][0] = q[0];
        pv[c][s][1] = q[1];
      }
    }
  }
  float v[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool in = t + c * kThreads < nch;
    unpack8(hv[c], v[c]);
    if constexpr (MODE != RN_EMBED) {
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {   // split order, as sum_splits8
        const bool sin = s < ks;
        acc[0] += sin ? pv[c][s][0].x : 0.f; acc[1] += sin ? pv[c][s][0].y : 0.f;
        acc[2] += sin ? pv[c][s][0].z : 0.f; acc[3] += sin ? pv[c][s][0].w : 0.f;
        acc[4] += sin ? pv[c][s][1].x : 0.f; acc[5] += sin ? pv[c][s][1].y : 0.f;
        acc[6] += sin ? pv[c][s][1].z : 0.f; acc[7] += sin ? pv[c][s][1].w : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[c][i] = MODE == RN_RESID_SCALED ? round_bf(v[c][i] + round_bf(round_bf(acc[i]) * alpha))
                                          : round_bf(v[c][i] + round_bf(acc[i]));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += in ? v[c][i] * v[c][i] : 0.f;
  }
  ss = block_sum(ss, red);
  const float rs = rsqrt_rn(ss / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = t + c * kThreads;
    if (ch >= nch) continue;
    st16(h_out + static_cast<size_t>(m) * H + 8 * ch, pack8(v[c]));
    float g[8], y[8];
    unpack8(gq[c], g);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = round_bf(round_bf(v[c][i] * rs) * g[i]);
    st16(xn + static_cast<size_t>(m) * H + 8 * ch, pack8(y));
  }
}

template <int MODE>
void launch_rows_norm(int m, hipStream_t stream, int ks, const uint16_t* table, const int64_t* ids, int64_t vocab,
                      const uint16_t* h_in, const float* part, uint16_t* h_out, const uint16_t* gamma, uint16_t* xn,
                      int M, int H, float eps, int* err, float alpha) {
  // one 8-element chunk per thread up to 2048 wide rows, two beyond
  auto go = [&](auto ksc, auto chc) {
    rows_norm_kernel<MODE, decltype(ksc)::value, decltype(chc)::value><<<m, kThreads, 0, stream>>>(
        table, ids, vocab, h_in, part, ks, h_out, gamma, xn, M, H, eps, err, alpha);
  };
  using K4 = std::integral_constant<int, 4>;
  using K8 = std::integral_constant<int, kMaxSplitsK>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, kRowChunks>;
  const bool one = H <= kThreads * 8;
  if (MODE == RN_EMBED || ks <= 4) {
    if (one) go(K4{}, C1{}); else go(K4{}, C2{});
  } else {
    if (one) go(K8{}, C1{}); else go(K8{}, C2{});
  }
}

// -------------------------------------------------------------- batch_sample
constexpr int kSampleThreads = 1024;

__global__ __launch_bounds__(kSampleThreads) void batch_sample_kernel(
    const float* __restrict__ bv, const int* __restrict__ bi, int nb, const int* inp,
    const int* plen, int64_t* ids, int* pos, int* sam, int nsteps, int* err) {
  __shared__ float rv[kSampleThreads / kWave];
  __shared__ int ri[kSampleThreads / kWave];
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  // the position and prompt length first, the next prompt id as soon as the
  // position is known: none of them waits behind the candidates' round trip
  const int p = pos[b];
  const int pl = plen[b];
  int nxt = 0;
  auto next_id = [&]() { nxt = inp[static_cast<size_t>(b) * nsteps + min(max(p + 1, 0), nsteps - 1)]; };
  const float* bvb = bv + static_cast<size_t>(b) * nb;
  const int* bib = bi + static_cast<size_t>(b) * nb;
  int best;
  if (nb <= 16 * kSampleThreads) {
    best = block_best_once<16>(bvb, bib, nb, rv, ri, next_id);
  } else {
    next_id();
    best = block_best(bvb, bib, nb, rv, ri);
  }
  if (t == 0) {
    if (p < 0 || p >= nsteps) {
      if (err) atomicExch(err, 2);
    } else {
      sam[static_cast<size_t>(b) * nsteps + p] = best;
      const bool prompt = (p + 1 < pl) && (p + 1 < nsteps);
      ids[b] = prompt ? static_cast<int64_t>(nxt) : static_cast<int64_t>(best);
      pos[b] = p + 1;
    }
  }
}

// ------------------------------------------------------------- top-p sampling
// The sampling step of MiniCPM3's run.py (examples/minicpm3_4b-cutedsl/run.py:29-47,
// `_sampler`): probabilities softmax(logits / T); ranked in descending order, a
// token is kept while the mass ranked before it is below top_p; one draw from
// the kept mass. One 512-thread block per sequence, thread t holding the
// vocabulary slice [t * per, t * per + per) in registers:
//   1. e = exp((logit - max logit) / T), Z = sum e;
//   2. the smallest f32 bit pattern tau with f(tau) = sum_{e > tau} e < top_p Z,
//      by binary search (positive floats order as their bit patterns): tau is
//      then itself a value of e, every e > tau is kept, and of the tokens equal
//      to tau those of tie rank r (in index order) with f(tau) + r tau < top_p Z
//      -- the prefix a stable descending sort would keep;
//   3. u in (0, 1) from a counter-based generator of (seed, sequence, position),
//      and the kept token where the running kept mass, in index order, first
//      exceeds u times the kept total (the distribution of a multinomial draw
//      over the ranked kept mass).
// Then the feed / advance of the greedy step: sam[b, pos] = the draw; the next
// input is the next prompt id while the prompt lasts, else the draw; pos + 1.
// Sums and scans run in a fixed order, so a draw is reproducible.
constexpr int kTopPThreads = 512;                      // two waves per SIMD: 256 registers a thread
constexpr int kTopPWaves = kTopPThreads / kWave;
constexpr int kTopPPer = 144;                          // vocabulary <= 73728

TFA_DEV uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Block-wide sum (every thread gets it), the waves' sums added in wave order.
// `slot` alternates between calls so that one barrier per call suffices.
TFA_DEV float topp_block_sum(float v, float (*red)[kTopPWaves], int& slot) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) red[slot][wid] = v;
  lds_barrier();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kTopPWaves; ++w) tot += red[slot][w];
  slot ^= 1;
  return tot;
}

TFA_DEV float topp_block_max(float v, float (*red)[kTopPWaves], int& slot) {
  v = wave_max(v);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) red[slot][wid] = v;
  lds_barrier();
  float m = red[slot][0];
#pragma unroll
  for (int w = 1; w < kTopPWaves; ++w) m = fmaxf(m, red[slot][w]);
  slot ^= 1;
  return m;
}

// Exclusive prefix sum over the threads in thread order (and the total).
TFA_DEV float topp_block_exscan(float v, float (*red)[kTopPWaves], int& slot, float& total) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  float inc = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const float o = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += o;
  }
  if (lane == kWave - 1) red[slot][wid] = inc;
  lds_barrier();
  float base = 0.f;
  total = 0.f;
#pragma unroll
  for (int w = 0; w < kTopPWaves; ++w) {
    if (w < wid) base += red[slot][w];
    total += red[slot][w];
  }
  slot ^= 1;
  return base + inc - v;
}

__global__ __launch_bounds__(kTopPThreads) void top_p_sample_kernel(
    const float* __restrict__ logits, int vocab, const float* __restrict__ params, const int64_t* __restrict__ seed,
    const int* inp, const int* plen, int64_t* ids, int* pos, int* sam, int nsteps, int* err) {
  __shared__ float red[2][kTopPWaves];
  __shared__ int s_pick, s_last;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  int slot = 0;
  const int p = pos[b];
  const int pl = plen[b];
  const int nxt = inp[static_cast<size_t>(b) * nsteps + min(max(p + 1, 0), nsteps - 1)];
  const float temp = params[0], top_p = params[1];
  const uint64_t sd = static_cast<uint64_t>(seed[0]);
  const int per = (vocab + kTopPThreads - 1) / kTopPThreads;
  const int i0 = t * per;
  const float* row = logits + static_cast<size_t>(b) * vocab;
  if (t == 0) {
    s_pick = -1;
    s_last = -1;
  }
  // 1. softmax numerators
  // every load from one per-lane base (immediate offsets, one memory round
  // trip): a slice that would run past the vocabulary is shifted back inside
  // it, and the slots that do not belong to this thread are masked once the
  // values are in
  float e[kTopPPer];
  const int nin = min(per, vocab - i0);         // this thread's tokens (<= 0 past the vocabulary)
  const int base = max(0, min(i0, vocab - kTopPPer));
  const int shift = i0 - base;                  // slot j holds token base + j
  const float* rb = row + base;
#pragma unroll
  for (int j = 0; j < kTopPPer; ++j) e[j] = rb[j];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < kTopPPer; ++j) {
    const int k = j - shift;                    // the slot's position in this thread's slice
    e[j] = k >= 0 && k < nin ? e[j] : -INFINITY;
    mx = fmaxf(mx, e[j]);
  }
  // exp((x - max x) / T) as exp2 of one product per token (the weights are
  // drawn from, not compared bit for bit)
  const float M = topp_block_max(mx, red, slot);
  const float c = 1.4426950408889634f / temp;
  float zs = 0.f;
#pragma unroll
  for (int j = 0; j < kTopPPer; ++j) {
    e[j] = e[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((e[j] - M) * c);
    zs += e[j];
  }
  const float Z = topp_block_sum(zs, red, slot);
  const float target = top_p * Z;
  // 2. the kept threshold: smallest tau with f(tau) < target (f(1.0) = 0)
  // e >= 0, so e > tau is an integer compare of the bit patterns; the select
  // is a mask of the sign of their difference (VALU bit operations only: no
  // per-element condition registers)
  auto mass_above = [&](float tau) __attribute__((always_inline)) {
    const int tb = __float_as_int(tau);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < kTopPPer; ++j) {
      const int eb = __float_as_int(e[j]);
      sum += __int_as_float(eb & ((tb - eb) >> 31));   // e if eb > tb, else +0
    }
    return topp_block_sum(sum, red, slot);
  };
  uint32_t lo = 0u, hi = 0x3F800000u;
  while (lo < hi) {   // uniform: every thread sees the same sums
    const uint32_t mid = lo + (hi - lo) / 2;
    if (mass_above(__uint_as_float(mid)) < target) hi = mid;
    else lo = mid + 1;
  }
  const float tau = __uint_as_float(lo);
  const float above = mass_above(tau);
  // tie rank of this thread's first token equal to tau, in index order
  float nt = 0.f;
#pragma unroll
  for (int j = 0; j < kTopPPer; ++j) {
    nt += (e[j] == tau && e[j] > 0.f) ? 1.f : 0.f;
    __builtin_amdgcn_sched_barrier(0);
  }
  float nties;
  float rank = topp_block_exscan(nt, red, slot, nties);
  // the kept weights, in place
  // (one element at a time: the scheduler may not hoist the compares, whose
  // masks would otherwise pile up and spill)
  float ks = 0.f;
  int last = -1;
#pragma unroll
  for (int j = 0; j < kTopPPer; ++j) {
    const float v = e[j];
    const bool tie = v == tau && v > 0.f;
    const bool keep = v > tau || (tie && above + rank * tau < target);
    rank += tie ? 1.f : 0.f;
    e[j] = keep ? v : 0.f;
    ks += e[j];
    last = keep && v > 0.f ? base + j : last;
    __builtin_amdgcn_sched_barrier(0);
  }
  float kept;
  const float before = topp_block_exscan(ks, red, slot, kept);
  if (last >= 0) atomicMax(&s_last, last);
  // 3. the draw
  const uint64_t r = mix64(sd ^ mix64(0x9E3779B97F4A7C15ull * static_cast<uint64_t>(b + 1) +
                                      static_cast<uint64_t>(static_cast<uint32_t>(p))));
  const float u = (static_cast<float>(r >> 40) + 0.5f) * (1.0f / 16777216.0f);
  const float goal = u * kept;
  if (ks > 0.f && goal >= before && goal < before + ks) {
    // the first kept token whose running mass passes the goal (branch-free)
    float acc = before;
    int pick = last;
    bool found = false;
#pragma unroll
    for (int j = 0; j < kTopPPer; ++j) {
      acc += e[j];
      const bool hit = !found && e[j] > 0.f && goal < acc;
      pick = hit ? base + j : pick;
      found = found || hit;
      __builtin_amdgcn_sched_barrier(0);
    }
    s_pick = pick;
  }
  lds_barrier();
  if (t == 0) {
    const int draw = s_pick >= 0 ? s_pick : s_last;   // u * kept rounded onto the total: the last kept token
    if (p < 0 || p >= nsteps || draw < 0) {
      if (err) atomicExch(err, 2);
    } else {
      sam[static_cast<size_t>(b) * nsteps + p] = draw;
      const bool prompt = (p + 1 < pl) && (p + 1 < nsteps);
      ids[b] = prompt ? static_cast<int64_t>(nxt) : static_cast<int64_t>(draw);
      pos[b] = p + 1;
    }
  }
}

}  // namespace

extern "C" {

int64_t tfa_skinny_blocks(int64_t n) { return (n + kGroupRows - 1) / kGroupRows; }

int tfa_skinny_gemm(const void* x, const void* w, int64_t m, int64_t n, int64_t k, int64_t ks,
                    int epilogue, float* part, void* act, float* logits, float* block_val,
                    int* block_idx, hipStream_t stream) {
  TFA_NONNULL(x);
  TFA_NONNULL(w);
  TFA_REQUIRE(m >= 1 && m <= kMaxTokens, TFA_ERR_SHAPE, "tfa_skinny_gemm: m=%lld not in [1, 32]", (long long)m);
  TFA_REQUIRE(n >= 1, TFA_ERR_SHAPE, "tfa_skinny_gemm: n=%lld must be positive", (long long)n);
  TFA_REQUIRE(ks >= 1 && k % (kWaves * kChunk * ks) == 0, TFA_ERR_SHAPE,
              "tfa_skinny_gemm: k=%lld must be a multiple of 256*ks (ks=%lld)", (long long)k, (long long)ks);
  TFA_ALIGN16(x);
  TFA_ALIGN16(w);
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.M = (int)m;
  a.N = (int)n;
  a.K = (int)k;
  a.ks = (int)ks;
  switch (epilogue) {
    case 0:
      TFA_NONNULL(part);
      a.part = part;
      return launch_skinny<SK_PARTIAL>(a, stream, "skinny_gemm_partial");
    case 1:
      TFA_NONNULL(act);
      TFA_REQUIRE(ks == 1 && n % 2 == 0, TFA_ERR_SHAPE, "tfa_skinny_gemm: swiglu needs ks=1 and even n");
      a.act = static_cast<uint16_t*>(act);
      return launch_skinny<SK_SWIGLU>(a, stream, "skinny_gemm_swiglu");
    case 2:
    case 3:
      TFA_NONNULL(block_val);
      TFA_NONNULL(block_idx);
      TFA_REQUIRE(ks == 1, TFA_ERR_SHAPE, "tfa_skinny_gemm: argmax needs ks=1");
      a.logits = logits;   // optional
      a.ngroups = (int)tfa_skinny_blocks(n);
      a.bv = block_val;
      a.bi = block_idx;
      if (epilogue == 3) return launch_skinny<SK_ARGMAX_BF16>(a, stream, "skinny_gemm_argmax_bf16");
      return launch_skinny<SK_ARGMAX>(a, stream, "skinny_gemm_argmax");
    default:
      return fail(TFA_ERR_ARG, "tfa_skinny_gemm: epilogue %d not in {0, 1, 2, 3}", epilogue);
  }
}

int64_t tfa_skinny_residual_blocks(int64_t n) { return (n + 31) / 32; }

int tfa_skinny_gemm_residual(const void* x, const void* w, int64_t m, int64_t n, int64_t k, const void* res,
                             void* h_out, float* ssq, hipStream_t stream) {
  TFA_NONNULL(x);
  TFA_NONNULL(w);
  TFA_NONNULL(res);
  TFA_NONNULL(h_out);
  TFA_NONNULL(ssq);
  TFA_REQUIRE(m >= 1 && m <= kMaxTokens, TFA_ERR_SHAPE, "tfa_skinny_gemm_residual: m=%lld not in [1, 32]", (long long)m);
  TFA_REQUIRE(n >= 1 && k % (kWaves * kChunk) == 0 && k > 0, TFA_ERR_SHAPE,
              "tfa_skinny_gemm_residual: n=%lld, k=%lld must be a positive multiple of 256", (long long)n, (long long)k);
  TFA_ALIGN16(x);
  TFA_ALIGN16(w);
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.M = (int)m;
  a.N = (int)n;
  a.K = (int)k;
  a.ks = 1;
  a.res = static_cast<const uint16_t*>(res);
  a.h_out = static_cast<uint16_t*>(h_out);
  a.ssq = ssq;
  return launch_skinny<SK_RESID_SSQ>(a, stream, "skinny_gemm_residual");
}

int tfa_skinny_gemm_norm_swiglu(const void* h, const void* w, int64_t m, int64_t n, int64_t k, const float* ssq,
                                int64_t nssq, const void* gamma, float eps, void* act, hipStream_t stream) {
  TFA_NONNULL(h);
  TFA_NONNULL(w);
  TFA_NONNULL(ssq);
  TFA_NONNULL(gamma);
  TFA_NONNULL(act);
  TFA_REQUIRE(m >= 1 && m <= kMaxTokens, TFA_ERR_SHAPE, "tfa_skinny_gemm_norm_swiglu: m=%lld not in [1, 32]", (long long)m);
  TFA_REQUIRE(n >= 2 && n % 2 == 0 && k % (kWaves * kChunk) == 0 && k > 0, TFA_ERR_SHAPE,
              "tfa_skinny_gemm_norm_swiglu: n=%lld must be even, k=%lld a positive multiple of 256", (long long)n,
              (long long)k);
  TFA_REQUIRE(nssq >= 1 && nssq <= 64, TFA_ERR_SHAPE, "tfa_skinny_gemm_norm_swiglu: %lld ssq rows not in [1, 64]",
              (long long)nssq);
  TFA_ALIGN16(h);
  TFA_ALIGN16(w);
  TFA_ALIGN16(gamma);
  SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.w = static_cast<const uint16_t*>(w);
  a.M = (int)m;
  a.N = (int)n;
  a.K = (int)k;
  a.ks = 1;
  a.act = static_cast<uint16_t*>(act);
  a.ssq_in = ssq;
  a.nssq = (int)nssq;
  a.gamma = static_cast<const uint16_t*>(gamma);
  a.eps = eps;
  return launch_skinny<SK_SWIGLU, true>(a, stream, "skinny_gemm_norm_swiglu");
}

int tfa_rows_norm(const void* table, const int64_t* ids, int64_t vocab, const void* h_in,
                  const float* part, int64_t ks, void* h_out, const void* gamma, void* xn,
                  int64_t m, int64_t hidden, float eps, int* err, hipStream_t stream) {
  TFA_NONNULL(h_out);
  TFA_NONNULL(gamma);
  TFA_NONNULL(xn);
  TFA_REQUIRE(m >= 0 && hidden > 0 && hidden % 8 == 0 && hidden <= kThreads * 8 * kRowChunks,
              TFA_ERR_SHAPE, "tfa_rows_norm: hidden %lld must be a multiple of 8, at most %d",
              (long long)hidden, kThreads * 8 * kRowChunks);
  TFA_ALIGN16(h_out);
  TFA_ALIGN16(xn);
  TFA_ALIGN16(gamma);
  if (table) {
    TFA_NONNULL(ids);
    TFA_REQUIRE(vocab > 0, TFA_ERR_SHAPE, "tfa_rows_norm: empty table");
  } else {
    TFA_NONNULL(h_in);
    TFA_NONNULL(part);
    TFA_REQUIRE(ks >= 1 && ks <= kMaxSplitsK, TFA_ERR_SHAPE, "tfa_rows_norm: ks %lld not in [1, %d]",
                (long long)ks, kMaxSplitsK);
  }
  if (m == 0) return TFA_OK;
  if (table)
    launch_rows_norm<RN_EMBED>((int)m, stream, 1, static_cast<const uint16_t*>(table), ids, vocab, nullptr, nullptr,
                               static_cast<uint16_t*>(h_out), static_cast<const uint16_t*>(gamma),
                               static_cast<uint16_t*>(xn), (int)m, (int)hidden, eps, err, 0.f);
  else
    launch_rows_norm<RN_RESID>((int)m, stream, (int)ks, nullptr, nullptr, 0, static_cast<const uint16_t*>(h_in), part,
                               static_cast<uint16_t*>(h_out), static_cast<const uint16_t*>(gamma),
                               static_cast<uint16_t*>(xn), (int)m, (int)hidden, eps, err, 0.f);
  return launched("rows_norm");
}

int tfa_rows_norm_scaled(const float* part, int64_t ks, const void* h_in, float alpha, void* h_out,
                         const void* gamma, void* xn, int64_t m, int64_t hidden, float eps, hipStream_t stream) {
  TFA_NONNULL(part);
  TFA_NONNULL(h_in);
  TFA_NONNULL(h_out);
  TFA_NONNULL(gamma);
  TFA_NONNULL(xn);
  TFA_REQUIRE(m >= 0 && hidden > 0 && hidden % 8 == 0 && hidden <= kThreads * 8 * kRowChunks,
              TFA_ERR_SHAPE, "tfa_rows_norm_scaled: hidden %lld must be a multiple of 8, at most %d",
              (long long)hidden, kThreads * 8 * kRowChunks);
  TFA_REQUIRE(ks >= 1 && ks <= kMaxSplitsK, TFA_ERR_SHAPE, "tfa_rows_norm_scaled: ks %lld not in [1, %d]",
              (long long)ks, kMaxSplitsK);
  TFA_ALIGN16(h_in);
  TFA_ALIGN16(h_out);
  TFA_ALIGN16(xn);
  TFA_ALIGN16(gamma);
  if (m == 0) return TFA_OK;
  launch_rows_norm<RN_RESID_SCALED>((int)m, stream, (int)ks, nullptr, nullptr, 0, static_cast<const uint16_t*>(h_in),
                                    part, static_cast<uint16_t*>(h_out), static_cast<const uint16_t*>(gamma),
                                    static_cast<uint16_t*>(xn), (int)m, (int)hidden, eps, nullptr, alpha);
  return launched("rows_norm_scaled");
}

int tfa_top_p_sample_step(const float* logits, int64_t vocab, int64_t batch, const float* params,
                          const int64_t* seed, const int* inp, const int* prompt_len, int64_t* ids, int* pos,
                          int* sam, int64_t nsteps, int* err, hipStream_t stream) {
  if (!logits || !params || !seed || !inp || !prompt_len || !ids || !pos || !sam)
    return fail(TFA_ERR_NULL, "tfa_top_p_sample_step: null pointer argument");
  TFA_REQUIRE(vocab > 0 && vocab <= (int64_t)kTopPThreads * kTopPPer, TFA_ERR_SHAPE,
              "tfa_top_p_sample_step: vocab %lld not in [1, %d]", (long long)vocab, kTopPThreads * kTopPPer);
  TFA_REQUIRE(batch > 0 && batch <= 65535 && nsteps > 0, TFA_ERR_SHAPE, "tfa_top_p_sample_step: empty shape");
  top_p_sample_kernel<<<(int)batch, kTopPThreads, 0, stream>>>(logits, (int)vocab, params, seed, inp, prompt_len,
                                                               ids, pos, sam, (int)nsteps, err);
  return launched("top_p_sample_step");
}

int tfa_batch_sample_step(const float* block_val, const int* block_idx, int64_t nblocks,
                          int64_t batch, const int* inp, const int* prompt_len, int64_t* ids,
                          int* pos, int* sam, int64_t nsteps, int* err, hipStream_t stream) {
  if (!block_val || !block_idx || !inp || !prompt_len || !ids || !pos || !sam)
    return fail(TFA_ERR_NULL, "tfa_batch_sample_step: null pointer argument");
  TFA_REQUIRE(nblocks > 0 && batch > 0 && nsteps > 0, TFA_ERR_SHAPE, "tfa_batch_sample_step: empty shape");
  batch_sample_kernel<<<(int)batch, kSampleThreads, 0, stream>>>(block_val, block_idx, (int)nblocks, inp,
                                                           prompt_len, ids, pos, sam, (int)nsteps, err);
  return launched("batch_sample_step");
}

}  // extern "C"
