// Multi-head latent attention (MLA) decode in the absorbed form, MiniCPM3-4B
// shapes: 40 heads, q_lora 768, kv_lora 256, rotary 32, nope 64, value 64.
//
// Per step and sequence the cache grows by one compressed entry -- the
// LoRA-normed latent c (256) and the rotated shared rope key (32) -- instead of
// 40 assembled keys and values. The query is absorbed: q_lat_h = W_UK_h^T q_nope_h,
// so scores are q_lat . c + q_rope . k_rope over the compressed cache, and the
// value up-projection W_UV_h is applied once to the weighted latent sum.
//
//   mla_prep      per sequence: reduce the [q_a | kv_c | k_rope] split-K
//                 partials, q_a -> LoRA norm (q_n for the q_b projection),
//                 kv_c -> LoRA norm -> latent cache slot pos, k_rope -> RoPE ->
//                 rope cache slot pos.
//   mla_q_absorb  per head: reduce the q_b partials, q_lat = bf16(W_UK^T q_nope)
//                 (f32 accumulate), q_rope -> RoPE; writes q_abs [B, H, 288].
//   mla_attn      per (split of 128*tiles positions, sequence), bf16 MFMA:
//                 S = q_abs . [c | k_rope]^T, online softmax in f32, O += P . c,
//                 each wave over its own positions and heads, merged at the end;
//                 writes the split's latent output (normalised by its own sum,
//                 bf16) with its max and sum.
//   mla_combine_up per (head, sequence): log-sum-exp merge of the splits into
//                 o_lat (f32), then bf16(W_UV o_lat) -> attn [B, H*64].
//   rows_residual out = bf16(res + bf16(bf16(sum_s part_s) * alpha)) -- the
//                 o_proj epilogue with MiniCPM3's scale_depth residual.
//
// Reference (jingchangshi/TileFoundry), non-absorbed: examples/minicpm3_4b-cutedsl/model.py:205-291
// (mla_attention), kernels/reference_ops.py:87-130 (rope_attend), kernels/cute_gemv.py:246-347
// (NORM_GEMV, NORM_GEMV_PAIR), kernels/cute_attention.py:56-200 (ROPE_ATTEND),
// kernels/cute_gemv.py:430-495 and reference_ops.py:63-65 (gemv_residual).
#include <float.h>

#include <mutex>
#include <type_traits>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kLat = 256;      // kv_lora_rank: the latent width
constexpr int kRope = 32;      // qk_rope_head_dim
constexpr int kQK = kLat + kRope;
constexpr int kNope = 64;      // qk_nope_head_dim
constexpr int kV = 64;         // v_head_dim
constexpr int kKvB = kNope + kV;   // rows of W_kv_b per head
constexpr int kHeadRows = 48;  // heads padded to three 16-row MFMA tiles
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxBatch = 32;
constexpr int kMaxSplits = 1024;
constexpr float kSlack = 8.0f;   // running-max headroom, log2 units

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

TFA_DEV bf16x8 as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

TFA_DEV void set_err(int* err, int code) {
  if (err) atomicExch(err, code);
}

// Rotate-half over 32 dims in bf16, each product and the sum landing: the
// torch spelling of reference_ops.py:99-109.
TFA_DEV float rope_bf(float x, float partner, float c, float s) {
  return round_bf(round_bf(x * c) + round_bf(partner * s));
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4
// of the 8-byte reads of lanes 4j + i / 4 (j = 0..3). Lane L reading row
// base + L / 4 at column col0 + 4 (L % 4) therefore receives
// C[base + j][col0 + i], j = 0..3 -- four consecutive rows of one column, the
// MFMA's K-major operand.
TFA_DEV uint2 ld_tr(const char* lds_byte) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_byte));
  return __builtin_bit_cast(uint2, v);
}

// ------------------------------------------------------------------ mla_prep
// One block per sequence. part: [ks, B, qa + 256 + 32] f32 split-K partials of
// x_n . [W_q_a; W_kv_a]^T; KS = ks, so that exactly the live partials are loaded.
template <int KS>
__global__ __launch_bounds__(kThreads) void mla_prep_kernel(
    const float* __restrict__ part, int ks, int B, int qa, const uint16_t* __restrict__ gq,
    const uint16_t* __restrict__ gkv, float eps, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int rope_rows, const int* __restrict__ pos,
    uint16_t* __restrict__ lat_cache, uint16_t* __restrict__ rope_cache, int cap,
    uint16_t* __restrict__ q_n, int* err) {
  __shared__ float sumsq[2][kWaves];
  __shared__ float kr[kRope];
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int row = qa + kLat + kRope;
  const size_t kstride = static_cast<size_t>(B) * row;
  const float* pb = part + static_cast<size_t>(b) * row;
  // Every load this thread needs goes out before any arithmetic (one memory
  // round trip), unconditionally at clamped indices: the position, both norm
  // scales, the split-K partials of its q_a, latent and rope values, and the
  // rope table row (behind the position's load only).
  const int p_raw = pos[b];
  uint32_t gqr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) gqr[j] = gq[min(t + kThreads * j, qa - 1)];
  const uint32_t gkr = gkv[t];
  float qp[4][KS], cp[KS], rp[KS];
  auto load_splits = [&](int i, float* v) __attribute__((always_inline)) {
#pragma unroll
    for (int sp = 0; sp < KS; ++sp) v[sp] = pb[static_cast<size_t>(sp) * kstride + i];
  };
#pragma unroll
  for (int j = 0; j < 4; ++j) load_splits(min(t + kThreads * j, qa - 1), qp[j]);
  load_splits(qa + t, cp);
  load_splits(qa + kLat + min(t, kRope - 1), rp);
  const bool p_ok = p_raw >= 0 && p_raw < cap && p_raw < rope_rows;
  const int pc = p_ok ? p_raw : 0;
  const uint32_t cr = cos_t[static_cast<size_t>(pc) * kRope + min(t, kRope - 1)];
  const uint32_t sr = sin_t[static_cast<size_t>(pc) * kRope + min(t, kRope - 1)];
  __builtin_amdgcn_sched_barrier(0);
  // the projection values land in bf16 (sum_splits' order)
  auto landed = [&](const float* v) __attribute__((always_inline)) {
    float acc = 0.f;
#pragma unroll
    for (int sp = 0; sp < KS; ++sp) acc += v[sp];
    return round_bf(acc);
  };
  float gqv[4], qv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in = t + kThreads * j < qa;
    gqv[j] = in ? bf2f(gqr[j]) : 0.f;
    qv[j] = in ? landed(qp[j]) : 0.f;
  }
  const float gk = bf2f(gkr);
  // q_a -> LoRA norm; kv_c -> LoRA norm (the latent); the rope slice
  const float cv = landed(cp);
  // every thread lands its (clamped) rope slice, so its loads are not sunk into
  // a branch; threads past the slice write the last value again, unchanged
  kr[min(t, kRope - 1)] = landed(rp);
  const float c = t < kRope && p_ok ? bf2f(cr) : 0.f;
  const float s = t < kRope && p_ok ? bf2f(sr) : 0.f;
  // both sums of squares in one block reduction (waves summed in order)
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) ss += qv[j] * qv[j];
  ss = wave_sum(ss);
  const float sk = wave_sum(cv * cv);
  const int lane = t & (kWave - 1), wid = t / kWave;
  if (lane == 0) {
    sumsq[0][wid] = ss;
    sumsq[1][wid] = sk;
  }
  __syncthreads();   // also publishes kr
  float tq = 0.f, tk = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    tq += sumsq[0][w];
    tk += sumsq[1][w];
  }
  const float rq = rsqrt_rn(tq / static_cast<float>(qa) + eps);
  const float rk = rsqrt_rn(tk / static_cast<float>(kLat) + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = t + kThreads * j;
    if (i < qa)
      q_n[static_cast<size_t>(b) * qa + i] = static_cast<uint16_t>(f2bf(round_bf(qv[j] * rq) * gqv[j]));
  }
  if (!p_ok) {
    if (t == 0) set_err(err, 6);
    return;
  }
  const int p = p_raw;
  lat_cache[(static_cast<size_t>(b) * cap + p) * kLat + t] = static_cast<uint16_t>(f2bf(round_bf(cv * rk) * gk));
  if (t < kRope) {
    const float x = kr[t];
    const float partner = t < kRope / 2 ? -kr[t + kRope / 2] : kr[t - kRope / 2];
    rope_cache[(static_cast<size_t>(b) * cap + p) * kRope + t] = static_cast<uint16_t>(f2bf(rope_bf(x, partner, c, s)));
  }
}

// -------------------------------------------------------------- mla_q_absorb
// One block per head. qpart: [ks, B, H*96] f32 split-K partials of
// q_n . W_q_b^T. w_kv_b: [H*128, 256] (out, in). Every load goes out first, 16
// bytes wide -- the positions, the head's W_UK (thread t: latent columns
// 8 (t % 32) .. + 7 of rows t / 32, t / 32 + 8, ...), the head's partials
// (16-byte pieces dealt over the block) -- so the block makes one memory round
// trip, and a second only for the rope rows of the positions. The partials
// land through LDS: each projection value is the sum of its splits in split
// order, landed in bf16. The absorbed query of eight sequences at a time: each
// thread's eight rows in order, then the row-group pairs (lanes l, l ^ 32) in
// registers, then the four waves in order through LDS. MAXB (1, 8 or 32) sizes
// the unrolled loads and passes.
template <int MAXB>
__global__ __launch_bounds__(kThreads) void mla_q_absorb_kernel(
    const float* __restrict__ qpart, int ks, int B, int H, const uint16_t* __restrict__ w_kv_b,
    const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t, int rope_rows,
    const int* __restrict__ pos, uint16_t* __restrict__ q_abs, int* err) {
  constexpr int kQH = kNope + kRope;                             // projection values per head
  constexpr int kQV = kQH / 4;                                   // their 16-byte pieces per (split, sequence)
  constexpr int kQLoads = (kMaxSplitsK * MAXB * kQV + kThreads - 1) / kThreads;
  constexpr int kPer = (MAXB * kQH + kThreads - 1) / kThreads;   // values per thread
  constexpr int kRopePer = (MAXB * kRope + kThreads - 1) / kThreads;
  constexpr int kGroup = MAXB < 8 ? MAXB : 8;                    // sequences per absorption pass
  constexpr int kRows = kNope / 8;                               // W_UK rows per thread
  __shared__ float4 qraw[kMaxSplitsK * MAXB * kQV];              // [split][sequence][piece]
  __shared__ float qn[MAXB][kNope];
  __shared__ float qr[MAXB][kRope];
  __shared__ float red[kWaves][kGroup][kLat];
  const int h = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(t / kWave);
  const int cc = lane & 31;          // latent columns 8cc .. 8cc + 7
  const int hi = lane >> 5;
  const int rg = 2 * wv + hi;        // W_UK rows rg + 8k
  const int qrow = H * kQH;
  const size_t kstride = static_cast<size_t>(B) * qrow;
  const int nq = ks * B * kQV;
  // 1. every load, none behind a branch (indices past the live range re-read
  //    the last piece, in bounds; their values are not used)
  int pr[kRopePer];
#pragma unroll
  for (int j = 0; j < kRopePer; ++j) pr[j] = pos[min((t + kThreads * j) / kRope, B - 1)];
  uint4 wk[kRows];
  const uint16_t* wuk = w_kv_b + (static_cast<size_t>(h) * kKvB + rg) * kLat + 8 * cc;
#pragma unroll
  for (int k = 0; k < kRows; ++k) wk[k] = ld16(wuk + static_cast<size_t>(8 * k) * kLat);
  // the partials in passes of kQPass pieces a thread (one pass up to batch 8)
  constexpr int kQPass = kQLoads < 6 ? kQLoads : 6;
  auto piece = [&](int j) __attribute__((always_inline)) {
    const int e = min(t + kThreads * j, nq - 1);
    const int sp = e / (B * kQV), r = e % (B * kQV);
    return *reinterpret_cast<const float4*>(qpart + sp * kstride + static_cast<size_t>(r / kQV) * qrow + h * kQH +
                                            4 * (r % kQV));
  };
  float4 qv[kQPass];
#pragma unroll
  for (int j = 0; j < kQPass; ++j) qv[j] = piece(j);
  uint32_t csr[kRopePer], snr[kRopePer];
#pragma unroll
  for (int j = 0; j < kRopePer; ++j) {
    const int e = t + kThreads * j;
    int p = pr[j];
    if (e < B * kRope && (p < 0 || p >= rope_rows)) {
      if (h == 0) set_err(err, 6);
      p = 0;
    }
    p = p < 0 || p >= rope_rows ? 0 : p;
    const int d = e % kRope;
    csr[j] = cos_t[static_cast<size_t>(p) * kRope + d];
    snr[j] = sin_t[static_cast<size_t>(p) * kRope + d];
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. the projection values land in bf16 (split order)
#pragma unroll
  for (int j = 0; j < kQPass; ++j)
    if (t + kThreads * j < nq) qraw[t + kThreads * j] = qv[j];
  for (int j0 = kQPass; j0 < kQLoads; j0 += kQPass) {
    float4 qw[kQPass];
#pragma unroll
    for (int j = 0; j < kQPass; ++j) qw[j] = piece(j0 + j);
#pragma unroll
    for (int j = 0; j < kQPass; ++j)
      if (t + kThreads * (j0 + j) < nq) qraw[t + kThreads * (j0 + j)] = qw[j];
  }
  lds_barrier();
  const float* qf = reinterpret_cast<const float*>(qraw);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = t + kThreads * j;
    if (e >= B * kQH) continue;
    const int b = e / kQH, i = e % kQH;
    float acc = 0.f;
#pragma unroll
    for (int sp = 0; sp < kMaxSplitsK; ++sp) acc += sp < ks ? qf[(sp * B + b) * kQH + i] : 0.f;
    if (i < kNope) qn[b][i] = round_bf(acc);
    else qr[b][i - kNope] = round_bf(acc);
  }
  float cs[kRopePer], sn[kRopePer];
#pragma unroll
  for (int j = 0; j < kRopePer; ++j) {
    cs[j] = bf2f(csr[j]);
    sn[j] = bf2f(snr[j]);
  }
  lds_barrier();
  // 3. q_abs[b, h, c] = bf16(sum_i qn[b][i] W_UK[i][c]), eight sequences a pass
  for (int b0 = 0; b0 < B; b0 += kGroup) {
    float acc[kGroup][8];
#pragma unroll
    for (int j = 0; j < kGroup; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      float w[8];
      unpack8(wk[k], w);
#pragma unroll
      for (int j = 0; j < kGroup; ++j) {
        const float q = qn[min(b0 + j, B - 1)][rg + 8 * k];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(q, w[e], acc[j][e]);
      }
    }
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[j][e]), __float_as_uint(acc[j][e]), false, false);
        acc[j][e] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
      }
      if (hi == 0) {
        *reinterpret_cast<float4*>(&red[wv][j][8 * cc]) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
        *reinterpret_cast<float4*>(&red[wv][j][8 * cc + 4]) = make_float4(acc[j][4], acc[j][5], acc[j][6], acc[j][7]);
      }
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const int b = b0 + j;
      if (b < B)
        q_abs[(static_cast<size_t>(b) * H + h) * kQK + t] =
            static_cast<uint16_t>(f2bf(((red[0][j][t] + red[1][j][t]) + red[2][j][t]) + red[3][j][t]));
    }
    lds_barrier();
  }
#pragma unroll
  for (int j = 0; j < kRopePer; ++j) {
    const int e = t + kThreads * j;
    if (e >= B * kRope) continue;
    const int b = e / kRope, d = e % kRope;
    const float partner = d < kRope / 2 ? -qr[b][d + kRope / 2] : qr[b][d - kRope / 2];
    q_abs[(static_cast<size_t>(b) * H + h) * kQK + kLat + d] =
        static_cast<uint16_t>(f2bf(rope_bf(qr[b][d], partner, cs[j], sn[j])));
  }
}

// ------------------------------------------------------------- mla_qb_absorb
// The q_b projection and the query absorption in one launch, two blocks per
// head (grid [H, 2]), both products on bf16 MFMA with f32 accumulation. Block
// (h, 0) projects the head's 64 nope rows of W_q_b, q_nope[b][i] =
// bf16(q_n[b] . W_q_b[96h + i]), and absorbs them, q_abs[b, h, c] =
// bf16(sum_i q_nope[b][i] W_UK_h[i][c]); block (h, 1) projects the 32 rope
// rows, lands them and rotates them at pos[b]. Every operand goes to LDS by
// DMA, all issued before any is read: the q_n rows, the block's weight rows
// (contiguous in W_q_b: 64 or 32 rows of 1536 bytes), then W_UK (64 rows of 512
// bytes). 16-byte piece s of a q_n or W_q_b row r sits at piece s ^ (r % 16) of
// its row, so an operand read (16 rows at one piece) is free of bank
// conflicts; the 32-byte chunks of W_UK row r are XOR-swizzled by
// (r % 4) + 4 ((r / 8) % 2), so the transpose reads of its operand (4 rows x
// 32 bytes per 16 lanes, row groups 8 apart) are too. Projection: wave w owns
// weight rows 16w .. 16w + 15 against every sequence, k-steps dealt over four
// accumulators; absorption: wave w owns latent columns 64w .. 64w + 63. NT:
// 16-sequence tiles (batch <= 16 NT); at NT = 2 the q_n rows take the LDS that
// W_UK has at NT = 1, so W_UK is loaded over the weight rows once the
// projection has read them.
// PREP (one sequence): the input is the f32 [q_a | kv_c | k_rope] partial of
// the LoRA-A projection instead of q_n. Every block brings q_a and gamma_q_a
// into LDS by DMA ahead of its weight rows and takes the LoRA norm while they
// stream (in mla_prep's order, so q_n is bit-equal to it); block (0, 1) also
// appends the normalised latent and the rotated rope key to the caches at
// pos[0] as mla_prep does.
constexpr int kQLora = 768;             // q_lora_rank: the K of the q_b projection
constexpr int kQbPieces = kQLora / 8;   // 16-byte pieces of a row
constexpr int kQnPitch = kNope + 8;     // landed q_nope row pitch, bf16 (144 bytes)
constexpr int kQaPieces = kQLora / 4;   // PREP: f32 q_a pieces, then gamma_q_a's kQbPieces
TFA_DEV int uk_slot(int row, int piece) { return piece ^ (2 * ((row & 3) | (((row >> 3) & 1) << 2))); }

struct QbArgs {
  const uint16_t* q_n;        // [B, 768] bf16 (not PREP)
  const float* part;          // PREP: [768 + 256 + 32] f32
  const uint16_t* gamma_q_a;  // PREP
  const uint16_t* gamma_kv_a; // PREP
  float eps;                  // PREP: the LoRA norms' eps
  uint16_t* lat_cache;        // PREP: [cap, 256]
  uint16_t* rope_cache;       // PREP: [cap, 32]
  int cap;
  const uint16_t* w_q_b;      // [H*96, 768]
  const uint16_t* w_kv_b;     // [H*128, 256]
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  int rope_rows;
  const int* pos;             // [B]
  uint16_t* q_abs;            // [B, H, 288]
  int* err;
  int B, H;
};

template <int NT, bool PREP>
__global__ __launch_bounds__(kThreads) void mla_qb_absorb_kernel(const QbArgs a) {
  static_assert(!PREP || NT == 1, "the prep form takes one sequence");
  constexpr int kQH = kNope + kRope;
  constexpr int kXRows = PREP ? 1 : 16 * NT;              // q_n rows in LDS
  constexpr int kXDma = 16 * NT * kQbPieces / kThreads;   // q_n DMAs per thread
  constexpr int kPreDma = 2;                              // PREP: q_a + gamma_q_a DMAs per thread
  constexpr int kUkDma = kNope * kLat / 8 / kThreads;     // W_UK DMAs per thread
  constexpr bool kUkEarly = NT == 1;                      // W_UK has LDS of its own
  constexpr int kRopePer = 16 * NT * kRope / kThreads;
  constexpr int kSteps = kQLora / 32;                     // projection k-steps
  constexpr int kBatch = 12;                              // k-steps whose operands are read at once
  static_assert(16 * NT * kQbPieces % kThreads == 0 && kRope * kQbPieces % kThreads == 0 &&
                    kNope * kLat / 8 % kThreads == 0 && kSteps % kBatch == 0, "loads split evenly");
  static_assert(kPreDma * kThreads >= kQaPieces + kQbPieces && kQLora == 3 * kThreads, "the prep's slots");
  static_assert(kWaves * 16 == kNope && kWaves * 64 == kLat, "one wave per 16 nope rows and 64 latent columns");
  __shared__ uint4 wl[kNope * kQbPieces];                 // W_q_b rows (at NT = 2 then W_UK)
  __shared__ uint4 xl[kXRows * kQbPieces];                // q_n rows
  __shared__ uint4 ukl[kUkEarly ? kNope * kLat / 8 : 1];  // W_UK rows (NT = 1)
  __shared__ uint4 pre[PREP ? kPreDma * kThreads : 1];    // PREP: q_a (f32) | gamma_q_a
  __shared__ float land[16 * NT * kQnPitch / 2];          // landed q_nope (bf16) or q_rope (f32)
  __shared__ float ssq[2][kWaves];                        // PREP: the q_a and latent norms' wave sums
  __shared__ float kr[kRope];                             // PREP: the landed rope key
  static_assert(sizeof(land) >= 16 * NT * kRope * 4, "q_rope fits the landing tile");
  uint16_t(*qnb)[kQnPitch] = reinterpret_cast<uint16_t(*)[kQnPitch]>(land);
  float(*qv)[kRope] = reinterpret_cast<float(*)[kRope]>(land);
  const int B = PREP ? 1 : a.B;
  const int H = a.H;
  const int h = blockIdx.x;
  const int part = blockIdx.y;   // 0: nope rows + absorption, 1: rope rows + rotation
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(t / kWave);
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const bool side = PREP && part == 1 && h == 0;   // the cache append

  // 1. every load: the rope table rows (part 1, in registers; the cache
  //    append's latent, rope-key and gamma values with them), then by DMA the
  //    q_n rows (rows past the batch re-read the last row) or q_a and
  //    gamma_q_a, the weight rows and (part 0, NT = 1) W_UK
  uint32_t csr[kRopePer], snr[kRopePer];
  int p_raw = 0;
  float cv = 0.f, krv = 0.f;
  uint32_t gkr = 0;
  if (part == 1) {
#pragma unroll
    for (int j = 0; j < kRopePer; ++j) {
      const int e = t + kThreads * j;
      int p = a.pos[min(e / kRope, B - 1)];
      if (j == 0) p_raw = p;
      if (e < B * kRope && (p < 0 || p >= a.rope_rows) && h == 0) set_err(a.err, 6);
      p = p < 0 || p >= a.rope_rows ? 0 : p;
      csr[j] = a.cos_t[static_cast<size_t>(p) * kRope + e % kRope];
      snr[j] = a.sin_t[static_cast<size_t>(p) * kRope + e % kRope];
    }
    if (side) {
      cv = a.part[kQLora + t];
      krv = a.part[kQLora + kLat + min(t, kRope - 1)];
      gkr = a.gamma_kv_a[t];
    }
  }
  const uint32_t xl0 = lds_offset(xl), wl0 = lds_offset(wl);
  if constexpr (PREP) {
    const uint32_t pre0 = lds_offset(pre);
#pragma unroll
    for (int i = 0; i < kPreDma; ++i) {
      const int q = kThreads * i + t;
      const void* src = q < kQaPieces ? static_cast<const void*>(a.part + 4 * q)
                                      : static_cast<const void*>(a.gamma_q_a + 8 * min(q - kQaPieces, kQbPieces - 1));
      lds_dma16(src, pre0 + (kThreads * i + kWave * w) * 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kXDma; ++i) {
      const int q = kThreads * i + t, r = q / kQbPieces, s = q % kQbPieces;
      lds_dma16(a.q_n + static_cast<size_t>(min(r, B - 1)) * kQLora + 8 * (s ^ (r & 15)),
                xl0 + (kThreads * i + kWave * w) * 16);
    }
  }
  const int ntile = part == 0 ? kNope / 16 : kRope / 16;
  const uint16_t* wsrc = a.w_q_b + (static_cast<size_t>(h) * kQH + part * kNope) * kQLora;
  for (int i = 0; i < ntile * 16 * kQbPieces / kThreads; ++i) {
    const int q = kThreads * i + t, r = q / kQbPieces, s = q % kQbPieces;
    lds_dma16_stream(wsrc + static_cast<size_t>(r) * kQLora + 8 * (s ^ (r & 15)), wl0 + (kThreads * i + kWave * w) * 16);
  }
  const uint16_t* uk_src = a.w_kv_b + static_cast<size_t>(h) * kKvB * kLat;
  auto issue_uk = [&](uint32_t dst0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kUkDma; ++i) {
      const int q = kThreads * i + t, r = q / (kLat / 8);
      lds_dma16_stream(uk_src + static_cast<size_t>(r) * kLat + 8 * uk_slot(r, q % (kLat / 8)),
                       dst0 + (kThreads * i + kWave * w) * 16);
    }
  };
  if (kUkEarly && part == 0) issue_uk(lds_offset(ukl));

  if constexpr (PREP) {
    // q_n = bf16(bf16(q_a * r) * gamma_q_a), q_a landed in bf16 (a one-split
    // sum, 0 + v); thread t sums its values t + 256j in order, then the wave,
    // then the four waves in order. The weight rows stay in flight.
    if (part == 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kNope * kQbPieces / kThreads + kUkDma));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(kRope * kQbPieces / kThreads));
    lds_barrier();
    const float* qa = reinterpret_cast<const float*>(pre);
    const uint16_t* gq = reinterpret_cast<const uint16_t*>(pre + kQaPieces);
    float qa3[3];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q = round_bf(0.f + (j < 3 ? qa[t + kThreads * j] : 0.f));
      if (j < 3) qa3[j] = q;
      ss += q * q;
    }
    ss = wave_sum(ss);
    float sk = 0.f;
    if (side) {
      cv = round_bf(0.f + cv);
      sk = wave_sum(cv * cv);
      if (t < kRope) kr[t] = round_bf(0.f + krv);
    }
    if (lane == 0) {
      ssq[0][w] = ss;
      ssq[1][w] = sk;
    }
    lds_barrier();
    float tq = 0.f;
#pragma unroll
    for (int w2 = 0; w2 < kWaves; ++w2) tq += ssq[0][w2];
    const float rq = rsqrt_rn(tq / static_cast<float>(kQLora) + a.eps);
    uint16_t* xq = reinterpret_cast<uint16_t*>(xl);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int i = t + kThreads * j;
      xq[i] = static_cast<uint16_t>(f2bf(round_bf(round_bf(qa3[j] * rq) * bf2f(gq[i]))));
    }
    if (side) {
      float tk = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) tk += ssq[1][w2];
      const float rk = rsqrt_rn(tk / static_cast<float>(kLat) + a.eps);
      if (p_raw < 0 || p_raw >= a.cap || p_raw >= a.rope_rows) {
        if (t == 0) set_err(a.err, 6);
      } else {
        a.lat_cache[static_cast<size_t>(p_raw) * kLat + t] = static_cast<uint16_t>(f2bf(round_bf(cv * rk) * bf2f(gkr)));
        if (t < kRope) {
          const float x = kr[t], partner = t < kRope / 2 ? -kr[t + kRope / 2] : kr[t - kRope / 2];
          a.rope_cache[static_cast<size_t>(p_raw) * kRope + t] =
              static_cast<uint16_t>(f2bf(rope_bf(x, partner, bf2f(csr[0]), bf2f(snr[0]))));
        }
      }
    }
  }
  if (kUkEarly && part == 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kUkDma));   // q_n and the weight rows landed
  else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  lds_barrier();

  // 2. the projection: C[sequence 16nt + 4g + r][row 16w + n16]; k-step ks
  //    reads piece 4ks + g of both operands (at PREP every lane reads row 0)
  f32x4 c[NT];
  if (w < ntile) {
    f32x4 acc[4][NT];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4* wrow = wl + (16 * w + n16) * kQbPieces;
#pragma unroll
    for (int k0 = 0; k0 < kSteps; k0 += kBatch) {
      uint4 bw[kBatch], ax[kBatch][NT];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int p = 4 * (k0 + j) + g;
        bw[j] = wrow[p ^ n16];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) ax[j][nt] = PREP ? xl[p] : xl[(16 * nt + n16) * kQbPieces + (p ^ n16)];
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[j & 3][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(ax[j][nt]), as_bf8(bw[j]), acc[j & 3][nt],
                                                                   0, 0, 0);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) c[nt] = (acc[0][nt] + acc[1][nt]) + (acc[2][nt] + acc[3][nt]);
    // landed: q_nope in bf16 (the absorption's operand), q_rope in f32
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * nt + 4 * g + r, col = 16 * w + n16;
        if (part == 0) qnb[row][col] = static_cast<uint16_t>(f2bf(c[nt][r]));
        else qv[row][col] = round_bf(c[nt][r]);
      }
  }
  if (part == 0) {
    if (!kUkEarly) {
      lds_barrier();   // every wave has read its weight rows: W_UK goes over them
      issue_uk(wl0);
    }
    // W_UK landed: the absorption reads it, and no DMA of the block may still be
    // writing LDS when it ends
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  lds_barrier();

  if (part == 1) {
    // 3b. q_rope rotated at the sequence's position
#pragma unroll
    for (int j = 0; j < kRopePer; ++j) {
      const int e = t + kThreads * j;
      if (e >= B * kRope) continue;
      const int b = e / kRope, d = e % kRope;
      const float partner = d < kRope / 2 ? -qv[b][d + kRope / 2] : qv[b][d - kRope / 2];
      a.q_abs[(static_cast<size_t>(b) * H + h) * kQK + kLat + d] =
          static_cast<uint16_t>(f2bf(rope_bf(qv[b][d], partner, bf2f(csr[j]), bf2f(snr[j]))));
    }
    return;
  }
  // 3a. q_abs[b, h, c] = bf16(sum_i q_nope[b][i] W_UK[i][c]): A = q_nope rows
  //     16bt + n16 (k = 32ks + 8g ..), B = W_UK by transpose reads of rows
  //     32ks + 8g + n16 / 4 (+ 4) at column col + 4 (n16 % 4)
  const char* uk = kUkEarly ? reinterpret_cast<const char*>(ukl) : reinterpret_cast<const char*>(wl);
  const char* qb = reinterpret_cast<const char*>(qnb);
#pragma unroll
  for (int bt = 0; bt < NT; ++bt) {
    uint4 aq[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      aq[ks] = *reinterpret_cast<const uint4*>(qb + (16 * bt + n16) * kQnPitch * 2 + (32 * ks + 8 * g) * 2);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = 64 * w + 16 * nt;
      const int cb = col + 4 * (n16 & 3);
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int r1 = 32 * ks + 8 * g + (n16 >> 2), r2 = r1 + 4;
        const uint2 v1 = ld_tr(uk + r1 * kLat * 2 + uk_slot(r1, cb / 8) * 16 + (cb % 8) * 2);
        const uint2 v2 = ld_tr(uk + r2 * kLat * 2 + uk_slot(r2, cb / 8) * 16 + (cb % 8) * 2);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(aq[ks]), as_bf8(make_uint4(v1.x, v1.y, v2.x, v2.y)),
                                                      acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = 16 * bt + 4 * g + r;
        if (b < B) a.q_abs[(static_cast<size_t>(b) * H + h) * kQK + col + n16] = static_cast<uint16_t>(f2bf(acc[r]));
      }
    }
  }
}

// ------------------------------------------------------------------ mla_attn
struct MlaAttnArgs {
  const uint16_t* q;     // [B, H, 288]: q_lat | rotated q_rope
  const uint16_t* lat;   // [B, cap, 256]
  const uint16_t* rk;    // [B, cap, 32]
  const int* wr;         // [B] newest slot: attend slots 0..wr[b]
  uint16_t* op;          // [B, ns, H, 256] split output / split sum (bf16)
  float* mp;             // [B, ns, H] split max
  float* lp;             // [B, ns, H] split sum
  int* err;
  int H, cap, ns, tiles;   // a split is `tiles` steps of kStep positions
  float scale;
  float scale_log2;   // scale * log2(e)
};

// Splits of 32 / 64 / 96 positions (the short-latency form for one sequence;
// splits of whole 128-position steps take mla_attn_heads_kernel below): a step
// is 32 positions in two LDS stages, filled by DMA. Wave mt -- three waves,
// one per head tile -- owns heads 16mt .. 16mt + 15 over the whole split with
// its own online-softmax state. One barrier per step publishes the step's
// rows and frees the other stage for the next step's DMA.
constexpr int kWaveRows = 32;
constexpr int kStepVm = 6;   // DMAs per wave per step: 2Q rows' latent and rope per wave
constexpr int kWaitVmStep = waitcnt_vm(kStepVm);
template <int Q>
struct AttnShape {
  static constexpr int waves = 3 * Q;
  static constexpr int step = Q * kWaveRows;
  static constexpr int lat_stage = step * kLat * 2;     // bytes
  static constexpr int stage_bytes = lat_stage + step * kRope * 2;
  static_assert(stage_bytes / (16 * kWave) == kStepVm * waves, "step DMA split evenly over the waves");
};
constexpr int kWaitVm0 = waitcnt_vm(0);

// Latent rows are 512 bytes of 32 16-byte chunks, stored XOR-swizzled by the
// row: the score operand reads (16 rows, one chunk) and the transpose reads of
// the value product (8 rows x 32 bytes per half-wave) then both hit 16
// distinct bank groups. The maps are involutions: slot <-> chunk.
TFA_DEV int lat_slot(int row, int chunk) { return chunk ^ (((row & 7) << 1) | ((row >> 3) & 1)); }
TFA_DEV int rope_slot(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

// Scores are computed transposed, S^T = [c | k_rope] . q^T (positions as MFMA
// rows, heads as columns): the accumulator of lane (head n16, row group g)
// then holds positions 4g + r of 16, which is exactly the K-slice lane
// (n16, g) supplies as the B operand of the value product O^T += C^T . P^T,
// so the weights never leave registers. K index 8g + i of that product is
// position 4g + i (i < 4) or 16 + 4g + i - 4 of the wave's 32.
template <int Q>
__global__ __launch_bounds__(3 * Q * kWave) __attribute__((amdgpu_waves_per_eu(3, 3)))
void mla_attn_kernel(const MlaAttnArgs a) {
  static_assert(Q == 1, "one 32-position quarter per step");
  constexpr int kAttnWaves = AttnShape<Q>::waves;
  constexpr int kStep = AttnShape<Q>::step;
  constexpr int kLatStage = AttnShape<Q>::lat_stage;
  constexpr int kStageBytes = AttnShape<Q>::stage_bytes;
  __shared__ uint4 smem[2 * kStageBytes / 16];   // two stages

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int u = wid / 3;    // position quarter (0: one quarter per step)
  const int mt = wid % 3;   // head tile
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const int s = blockIdx.x;
  const int b = blockIdx.y;

  int last = __builtin_amdgcn_readfirstlane(a.wr[b]);
  if (last < 0 || last >= a.cap) {
    if (s == 0 && threadIdx.x == 0) set_err(a.err, 4);
    last = last < 0 ? -1 : a.cap - 1;
  }
  const int n = last + 1;
  const int pos0 = s * kStep * a.tiles;
  if (pos0 >= n) return;
  const int nsteps = min(a.tiles, (n - pos0 + kStep - 1) / kStep);
  const uint16_t* lat = a.lat + static_cast<size_t>(b) * a.cap * kLat;
  const uint16_t* rk = a.rk + static_cast<size_t>(b) * a.cap * kRope;
  const char* lds = reinterpret_cast<const char*>(smem);
  const uint32_t lds0 = lds_offset(smem);

  // Step t's rows into stage st, DMAs 6 wid .. 6 wid + 5 of the step: latent
  // DMA j lands rows 2j, 2j + 1 (lane L at row 2j + L/32, slot L%32, so it
  // fetches chunk lat_slot(row, slot)); rope DMA j - 64 lands 16 rows. Rows
  // past the context load the last live row instead (finite data; their
  // weight is zero), also for a step past the end.
  auto issue = [&](int t, int st) __attribute__((always_inline)) {
    const int p0 = pos0 + kStep * t;
#pragma unroll
    for (int i = 0; i < kStepVm; ++i) {
      const int j = kStepVm * wid + i;
      if (j < kStep / 2) {
        const int row = 2 * j + (lane >> 5);
        const int p = min(p0 + row, n - 1);
        lds_dma16_stream(lat + static_cast<size_t>(p) * kLat + 8 * lat_slot(row, lane & 31),
                  lds0 + st * kStageBytes + j * 16 * kWave);
      } else {
        const int row = 16 * (j - kStep / 2) + (lane >> 2);
        const int p = min(p0 + row, n - 1);
        lds_dma16_stream(rk + static_cast<size_t>(p) * kRope + 8 * rope_slot(row, lane & 3),
                  lds0 + st * kStageBytes + kLatStage + (j - kStep / 2) * 16 * kWave);
      }
    }
  };

  // q^T operands, resident: lane (n16, g) holds q[head 16mt + n16][32ks + 8g ..
  // +7] (padding heads repeat the last head; their results are never stored).
  // Loaded before any DMA: the compiler's own wait for them, at their first
  // use in step 0, is then the only wait it places.
  uint4 qop[9];
  {
    const uint16_t* qrow = a.q + (static_cast<size_t>(b) * a.H + min(16 * mt + n16, a.H - 1)) * kQK + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) qop[ks] = ld16(qrow + 32 * ks);
  }
  issue(0, 0);
  // The DMAs are invisible to the compiler, so its own wait for the q loads
  // (issued before them) also waits for every DMA behind them. With a second
  // step that wait covers both stages; a one-step split issues nothing more,
  // so step 0 waits for its own rows only (one sequence at 300 positions:
  // 8.3 -> 7.8 us).
  if (nsteps > 1) issue(1, 1);

  // Lane byte offsets into a stage (the lat_slot swizzle worked out so that
  // the rest of each address is an immediate). Score operand (ks, pt): row
  // 32u + 16pt + n16, chunk 4ks + g, at so[ks % 4] + 256 (ks / 4) + 8192 pt.
  const int fs = ((n16 & 7) << 1) | (n16 >> 3);
  uint32_t so[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    so[j] = (kWaveRows * u + n16) * 2 * kLat + 16 * (g ^ (fs & 3)) + 64 * (j ^ (fs >> 2));
  const uint32_t ro = kLatStage + (kWaveRows * u + n16) * 2 * kRope + 16 * (g ^ ((n16 >> 2) & 3));   // + 1024 pt
  // value operand ct: rows r1 = 32u + 4g + n16/4 and r1 + 16, columns
  // 16ct + 4 (n16 % 4), at to[ct % 8] + 256 (ct / 8) (+ 8192 for r1 + 16)
  const int r1 = 4 * g + (n16 >> 2);
  const int f1 = ((r1 & 7) << 1) | ((r1 >> 3) & 1);
  uint32_t to[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    to[j] = (kWaveRows * u + r1) * 2 * kLat + 16 * (((n16 & 3) >> 1) ^ (f1 & 1)) + 8 * (n16 & 1) +
            32 * (j ^ (f1 >> 1));

  // running state of head 16mt + n16 (the same in the lane's four row groups;
  // l_run sums only the lane's own positions)
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[16];   // O^T[latent column 16ct + 4g + r][head 16mt + n16]
#pragma unroll
  for (int ct = 0; ct < 16; ++ct) o[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  bool started = false;
  const bool live_tile = 16 * mt < a.H;

  auto step = [&](int t, const char* stage) __attribute__((always_inline)) {
    const int pb = pos0 + kStep * t + kWaveRows * u;
    if (!live_tile || pb >= n) return;   // no live position or head in this wave's block
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < 9; ++ks)
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        const uint4 aop = ks < 8 ? *reinterpret_cast<const uint4*>(stage + so[ks & 3] + 256 * (ks >> 2) + 8192 * pt)
                                 : *reinterpret_cast<const uint4*>(stage + ro + 1024 * pt);
        sacc[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(aop), as_bf8(qop[ks]), sacc[pt], 0, 0, 0);
      }
    // scores in log2 units (the scale folded in); masked positions are -inf
    float sv[2][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int pt = 0; pt < 2; ++pt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[pt][r] = pb + 16 * pt + 4 * g + r < n ? sacc[pt][r] * a.scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, sv[pt][r]);
      }
    // online softmax: the running max (log2 units) is only raised -- and O
    // rescaled -- when some head's block max passes it by more than kSlack,
    // so the weights exp2(s - m) stay <= 2^kSlack. Position pb is live, so
    // every head's block max is finite.
    tmax = rows4_max(tmax);
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kSlack) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // 0 while m_run is -inf
      l_run *= alpha;
      m_run = m_new;
      if (started) {
#pragma unroll
        for (int ct = 0; ct < 16; ++ct) o[ct] *= alpha;
      }
      started = true;
    }
    float e[2][4];
#pragma unroll
    for (int pt = 0; pt < 2; ++pt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        e[pt][r] = __builtin_amdgcn_exp2f(sv[pt][r] - m_run);   // masked: exp2(-inf) = 0
        l_run += e[pt][r];
      }
    // P^T operand: bf16 weights of positions 4g + {0..3, 16..19}
    const uint4 pop = make_uint4(pack_bf(e[0][0], e[0][1]), pack_bf(e[0][2], e[0][3]), pack_bf(e[1][0], e[1][1]),
                                 pack_bf(e[1][2], e[1][3]));
    // O^T += C^T . P^T over the wave's 32 positions
#pragma unroll
    for (int ct = 0; ct < 16; ++ct) {
      const uint2 v1 = ld_tr(stage + to[ct & 7] + 256 * (ct >> 3));
      const uint2 v2 = ld_tr(stage + to[ct & 7] + 256 * (ct >> 3) + 16 * 2 * kLat);
      o[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(make_uint4(v1.x, v1.y, v2.x, v2.y)), as_bf8(pop), o[ct],
                                                       0, 0, 0);
    }
  };

  // step 0 (step 1 is in flight behind it); from step 1 on, the next step's
  // DMA goes out once every wave is past the barrier, i.e. done with the
  // stage it refills
  if (nsteps > 1)
    __builtin_amdgcn_s_waitcnt(kWaitVmStep);
  else
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  block_barrier();
  step(0, lds);
  for (int t = 1; t < nsteps; ++t) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    block_barrier();
    if (t + 1 < nsteps) issue(t + 1, (t + 1) & 1);
    step(t, lds + (t & 1) * kStageBytes);
  }

  // the wave holds its head tile's whole split
  const float lsum = rows4_sum(l_run);
  const float fself = 1.0f / lsum;
  const size_t orow = (static_cast<size_t>(b) * a.ns + s) * a.H;
  const int h = 16 * mt + n16;
  if (h < a.H) {
#pragma unroll
    for (int ct = 0; ct < 16; ++ct) {
      const f32x4 acc = o[ct] * fself;
      *reinterpret_cast<uint2*>(a.op + (orow + h) * kLat + 16 * ct + 4 * g) =
          make_uint2(pack_bf(acc[0], acc[1]), pack_bf(acc[2], acc[3]));
    }
    if (g == 0) {
      a.mp[orow + h] = m_run * 0.6931471805599453f;   // natural-log units
      a.lp[orow + h] = lsum;
    }
  }
}

// Splits of whole 128-position steps: eight waves, two per SIMD, each holding
// the query of all 48 (padded) heads. Wave w scores positions 16w .. 16w + 15
// of the step against every head, so each cache row is read from LDS once for
// the scores (three times when waves own head tiles). The per-head maxima of
// the eight position groups meet in LDS, so every wave raises the same running
// max; the bf16 weights go to LDS in the value product's operand layout; and
// wave w accumulates latent columns 32w .. 32w + 31 of every head over all 128
// positions. Its O is then final for those columns: only the per-head sums are
// combined at the end, with no merge of partial O.
constexpr int kHW = 8;
constexpr int kHRows = 16;                       // positions scored per wave per step
constexpr int kHStep = kHW * kHRows;             // 128
constexpr int kHLatStage = kHStep * kLat * 2;
constexpr int kHStageBytes = kHLatStage + kHStep * kRope * 2;
constexpr int kHLatDma = kHStep / 2 / kHW;       // latent DMAs per wave per step (two rows each)
constexpr int kHRopeDma = kHStep / 16 / kHW;     // rope DMAs per wave per step (16 rows each)
constexpr int kHStepVm = kHLatDma + kHRopeDma;
static_assert(kHStepVm * kHW * 16 * kWave == kHStageBytes, "step DMA split evenly over the waves");
constexpr int kHQDma = 4;                        // query DMAs per wave: 32 KB >= 48 heads x 576 B
static_assert(kHQDma * kHW * 16 * kWave >= kHeadRows * kQK * 2 && kHQDma * kHW * 16 * kWave <= kHStageBytes,
              "the query fits the second stage");
static_assert(kHQDma + 2 * kHStepVm <= 63, "the DMAs in flight fit the vmcnt counter");
constexpr int kHWaitVmStep = waitcnt_vm(kHStepVm);
static_assert(kHW == 8, "a head's eight wave maxima / sums are two float4 in LDS");

__global__ __launch_bounds__(kHW * kWave) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mla_attn_heads_kernel(const MlaAttnArgs a) {
  __shared__ uint4 smem[2 * kHStageBytes / 16];   // two stages of cache rows
  __shared__ uint2 pw[kHStep / 32][3][kWave][2];  // P^T operands [32-position group][head tile][lane][half]
  __shared__ float4 sx[kHeadRows][kHW / 4];       // per-head maxima of the waves, at the end their sums

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const int s = blockIdx.x;
  const int b = blockIdx.y;

  int last = __builtin_amdgcn_readfirstlane(a.wr[b]);
  if (last < 0 || last >= a.cap) {
    if (s == 0 && threadIdx.x == 0) set_err(a.err, 4);
    last = last < 0 ? -1 : a.cap - 1;
  }
  const int n = last + 1;
  const int pos0 = s * kHStep * a.tiles;
  if (pos0 >= n) return;
  const int nsteps = min(a.tiles, (n - pos0 + kHStep - 1) / kHStep);
  const uint16_t* lat = a.lat + static_cast<size_t>(b) * a.cap * kLat;
  const uint16_t* rk = a.rk + static_cast<size_t>(b) * a.cap * kRope;
  const char* lds = reinterpret_cast<const char*>(smem);
  const uint32_t lds0 = lds_offset(smem);

  // step t's rows into stage st: latent DMA j lands rows 2j, 2j + 1 (wave w
  // issues j = 8w .. 8w + 7), rope DMA j rows 16j .. 16j + 15 (wave w: j = w).
  // Rows past the context load the last live row (finite; their weight is 0).
  auto issue = [&](int t, int st) __attribute__((always_inline)) {
    const int p0 = pos0 + kHStep * t;
#pragma unroll
    for (int i = 0; i < kHLatDma; ++i) {
      const int j = kHLatDma * w + i;
      const int row = 2 * j + (lane >> 5);
      const int p = min(p0 + row, n - 1);
      lds_dma16_stream(lat + static_cast<size_t>(p) * kLat + 8 * lat_slot(row, lane & 31),
                       lds0 + st * kHStageBytes + j * 16 * kWave);
    }
#pragma unroll
    for (int i = 0; i < kHRopeDma; ++i) {
      const int j = kHRopeDma * w + i;
      const int row = 16 * j + (lane >> 2);
      const int p = min(p0 + row, n - 1);
      lds_dma16_stream(rk + static_cast<size_t>(p) * kRope + 8 * rope_slot(row, lane & 3),
                       lds0 + st * kHStageBytes + kHLatStage + j * 16 * kWave);
    }
  };

  // The query rows of the sequence (H x 576 bytes) go by DMA into the second
  // stage, then to registers, before that stage is filled. Every load of the
  // kernel is then a DMA the waits below count exactly: step 0 starts once its
  // own rows have landed, with step 1's still in flight behind them (a query
  // held by register loads would be waited for by the compiler with a wait
  // for every load in flight, step 1's rows included).
  {
    const int qbytes = a.H * kQK * 2;
    const char* qseq = reinterpret_cast<const char*>(a.q + static_cast<size_t>(b) * a.H * kQK);
#pragma unroll
    for (int i = 0; i < kHQDma; ++i) {
      const int j = kHW * i + w;   // 1 KB piece j of the query rows (pieces past the end re-read the last 16 bytes)
      lds_dma16(qseq + min(1024 * j + 16 * lane, qbytes - 16), lds0 + kHStageBytes + j * 16 * kWave);
    }
  }
  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(kHStepVm));   // this wave's query pieces landed
  lds_barrier();
  // q^T operands of the three head tiles, resident: lane (n16, g) holds
  // q[head 16mt + n16][32ks + 8g .. +7] (padding heads repeat the last head)
  uint4 qop[3][9];
#pragma unroll
  for (int mt = 0; mt < 3; ++mt) {
    const char* qrow = lds + kHStageBytes + min(16 * mt + n16, a.H - 1) * kQK * 2 + 16 * g;
#pragma unroll
    for (int ks = 0; ks < 9; ++ks) qop[mt][ks] = *reinterpret_cast<const uint4*>(qrow + 64 * ks);
  }
  lds_barrier();   // every wave has its query: the second stage is free
  if (nsteps > 1) issue(1, 1);

  // score operand ks of wave w: row 16w + n16, chunk 4ks + g
  const int fs = ((n16 & 7) << 1) | (n16 >> 3);
  uint32_t so[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) so[j] = (kHRows * w + n16) * 2 * kLat + 16 * (g ^ (fs & 3)) + 64 * (j ^ (fs >> 2));
  const uint32_t ro = kHLatStage + (kHRows * w + n16) * 2 * kRope + 16 * (g ^ ((n16 >> 2) & 3));
  // value operand of column tile 2w + c over 32-position group kk: rows 32kk +
  // r1 and 32kk + r1 + 16 (r1 = 4g + n16 / 4), columns 16 (2w + c) + 4 (n16 %
  // 4), at tw[c] + 16384 kk (+ 8192 for the second row)
  const int r1 = 4 * g + (n16 >> 2);
  const int f1 = ((r1 & 7) << 1) | ((r1 >> 3) & 1);
  uint32_t tw[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int ct = 2 * w + c;
    tw[c] = r1 * 2 * kLat + 16 * (((n16 & 3) >> 1) ^ (f1 & 1)) + 8 * (n16 & 1) + 32 * ((ct & 7) ^ (f1 >> 1)) +
            256 * (ct >> 3);
  }

  // running state of head 16mt + n16 (the same in every wave; l_run sums only
  // this lane's own positions)
  float m_run[3] = {-INFINITY, -INFINITY, -INFINITY};
  float l_run[3] = {0.f, 0.f, 0.f};
  bool started[3] = {false, false, false};
  f32x4 o[3][2];   // O^T[latent column 16 (2w + c) + 4g + r][head 16mt + n16]
#pragma unroll
  for (int mt = 0; mt < 3; ++mt) o[mt][0] = o[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int t, const char* stage) __attribute__((always_inline)) {
    const int pb = pos0 + kHStep * t + kHRows * w;
    const bool live = pb < n;   // some position of this wave's 16 is in the context
    f32x4 sacc[3];
#pragma unroll
    for (int mt = 0; mt < 3; ++mt) sacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (live) {
#pragma unroll
      for (int ks = 0; ks < 9; ++ks) {
        const uint4 aop = ks < 8 ? *reinterpret_cast<const uint4*>(stage + so[ks & 3] + 256 * (ks >> 2))
                                 : *reinterpret_cast<const uint4*>(stage + ro);
#pragma unroll
        for (int mt = 0; mt < 3; ++mt)
          sacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(aop), as_bf8(qop[mt][ks]), sacc[mt], 0, 0, 0);
      }
    }
    // scores in log2 units; masked positions (and a whole dead wave) -inf
    float sv[3][4];
#pragma unroll
    for (int mt = 0; mt < 3; ++mt) {
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[mt][r] = live && pb + 4 * g + r < n ? sacc[mt][r] * a.scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, sv[mt][r]);
      }
      tmax = rows4_max(tmax);
      if (g == 0) reinterpret_cast<float*>(sx[16 * mt + n16])[w] = tmax;
    }
    lds_barrier();
    // the step max of each head over the eight groups; the running max is
    // raised (and O rescaled) only when some head of the tile passes it by
    // kSlack -- the same decision in every wave, which read the same maxima
#pragma unroll
    for (int mt = 0; mt < 3; ++mt) {
      const int h = 16 * mt + n16;
      const float4 x0 = sx[h][0], x1 = sx[h][1];
      const float smax = fmaxf(fmaxf(fmaxf(x0.x, x0.y), fmaxf(x0.z, x0.w)), fmaxf(fmaxf(x1.x, x1.y), fmaxf(x1.z, x1.w)));
      if (__builtin_amdgcn_ballot_w64(smax > m_run[mt] + kSlack) != 0) {
        const float m_new = fmaxf(m_run[mt], smax);
        const float alpha = __builtin_amdgcn_exp2f(m_run[mt] - m_new);   // 0 while m_run is -inf
        l_run[mt] *= alpha;
        m_run[mt] = m_new;
        if (started[mt]) {
          o[mt][0] *= alpha;
          o[mt][1] *= alpha;
        }
        started[mt] = true;
      }
      float e[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        e[r] = __builtin_amdgcn_exp2f(sv[mt][r] - m_run[mt]);   // masked: exp2(-inf) = 0
        l_run[mt] += e[r];
      }
      // half (w % 2) of the P^T operand of group w / 2: bf16 weights of
      // positions 4g .. 4g + 3 of this wave's 16 (all zero past the context)
      pw[w >> 1][mt][lane][w & 1] = make_uint2(pack_bf(e[0], e[1]), pack_bf(e[2], e[3]));
    }
    lds_barrier();
    // O^T += C^T . P^T over the step's four 32-position groups, this wave's 32 columns
#pragma unroll
    for (int kk = 0; kk < kHStep / 32; ++kk) {
      uint4 aop[2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint2 v1 = ld_tr(stage + tw[c] + 16384 * kk);
        const uint2 v2 = ld_tr(stage + tw[c] + 16384 * kk + 8192);
        aop[c] = make_uint4(v1.x, v1.y, v2.x, v2.y);
      }
#pragma unroll
      for (int mt = 0; mt < 3; ++mt) {
        const uint4 pop = *reinterpret_cast<const uint4*>(&pw[kk][mt][lane][0]);
#pragma unroll
        for (int c = 0; c < 2; ++c)
          o[mt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(aop[c]), as_bf8(pop), o[mt][c], 0, 0, 0);
      }
    }
  };

  // the next step's DMA goes out once every wave is past the step barrier,
  // i.e. done with the stage it refills
  if (nsteps > 1)
    __builtin_amdgcn_s_waitcnt(kHWaitVmStep);
  else
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  block_barrier();
  step(0, lds);
  for (int t = 1; t < nsteps; ++t) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    block_barrier();
    if (t + 1 < nsteps) issue(t + 1, (t + 1) & 1);
    step(t, lds + (t & 1) * kHStageBytes);
  }

  // the per-head sums of the eight groups (every wave is past the last maxima
  // read, so sx is free), in group order; each wave stores its own columns
#pragma unroll
  for (int mt = 0; mt < 3; ++mt) {
    const float lw = rows4_sum(l_run[mt]);
    if (g == 0) reinterpret_cast<float*>(sx[16 * mt + n16])[w] = lw;
  }
  lds_barrier();   // every wave is past its last stage read: the stages are free
  // the normalised split output, through LDS so that each store instruction
  // writes 1 KB of whole head rows (rows padded to 528 bytes: the 16 heads of a
  // lane group land on distinct banks)
  constexpr int kOPitch = kLat + 8;
  static_assert(kHeadRows * kOPitch * 2 <= kHStageBytes, "the split output fits a stage");
  uint16_t* obuf = reinterpret_cast<uint16_t*>(smem);
  const size_t orow = (static_cast<size_t>(b) * a.ns + s) * a.H;
#pragma unroll
  for (int mt = 0; mt < 3; ++mt) {
    const int h = 16 * mt + n16;
    const float4 x0 = sx[h][0], x1 = sx[h][1];
    const float lsum = ((((((x0.x + x0.y) + x0.z) + x0.w) + x1.x) + x1.y) + x1.z) + x1.w;   // wave order
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const f32x4 acc = o[mt][c] * inv;
      *reinterpret_cast<uint2*>(obuf + h * kOPitch + 16 * (2 * w + c) + 4 * g) =
          make_uint2(pack_bf(acc[0], acc[1]), pack_bf(acc[2], acc[3]));
    }
    if (w == 0 && g == 0 && h < a.H) {
      a.mp[orow + h] = m_run[mt] * 0.6931471805599453f;   // natural-log units
      a.lp[orow + h] = lsum;
    }
  }
  lds_barrier();
  // 16-byte piece i of the H x 512-byte split output (consecutive heads are
  // consecutive rows of op)
  for (int i = threadIdx.x; i < a.H * (kLat / 8); i += kHW * kWave) {
    const int h = i / (kLat / 8), ch = i % (kLat / 8);
    *reinterpret_cast<uint4*>(a.op + (orow + h) * kLat + 8 * ch) =
        *reinterpret_cast<const uint4*>(obuf + h * kOPitch + 8 * ch);
  }
}

// ------------------------------------------------------------ mla_combine_up
// One block per (head, sequence): w_s = l_s e^(m_s - M), o_lat = sum_s w_s op_s /
// sum_s w_s (f32), then attn[b, h*64 + v] = bf16(sum_c W_UV[h][v][c] o_lat[c]).
__global__ __launch_bounds__(kThreads) void mla_combine_up_kernel(
    const uint16_t* __restrict__ op, const float* __restrict__ mp, const float* __restrict__ lp,
    const int* __restrict__ wr, int ns, int split, int H, int cap, const uint16_t* __restrict__ w_kv_b,
    uint16_t* __restrict__ attn) {
  __shared__ float wgt[kMaxSplits];
  __shared__ float olat[kLat];
  __shared__ float wave_max_s[kWaves];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  int last = wr[b];
  last = last < 0 ? 0 : (last >= cap ? cap - 1 : last);
  const int nsa = min(ns, last / split + 1);
  const size_t srow = static_cast<size_t>(b) * ns * H + h;   // (b, s=0, h)
  float mx = -INFINITY;
  for (int s = t; s < nsa; s += kThreads) mx = fmaxf(mx, mp[srow + static_cast<size_t>(s) * H]);
  mx = wave_max(mx);
  if ((t & (kWave - 1)) == 0) wave_max_s[t / kWave] = mx;
  lds_barrier();
  const float M = fmaxf(fmaxf(wave_max_s[0], wave_max_s[1]), fmaxf(wave_max_s[2], wave_max_s[3]));
  lds_barrier();
  for (int s = t; s < nsa; s += kThreads) {
    const size_t i = srow + static_cast<size_t>(s) * H;
    wgt[s] = lp[i] * expf(mp[i] - M);
  }
  lds_barrier();
  float L = 0.f, acc = 0.f;
  for (int s = 0; s < nsa; ++s) {
    L += wgt[s];
    acc = fmaf(wgt[s], bf2f(op[(srow + static_cast<size_t>(s) * H) * kLat + t]), acc);
  }
  olat[t] = acc / L;
  lds_barrier();
  // value row v = t / 4, latent quarter q = t % 4
  const int v = t >> 2, q = t & 3;
  const uint16_t* wrow = w_kv_b + (static_cast<size_t>(h) * kKvB + kNope + v) * kLat + 64 * q;
  float d = 0.f;
#pragma unroll
  for (int c8 = 0; c8 < 8; ++c8) {
    float w8[8];
    unpack8(ld16(wrow + 8 * c8), w8);
#pragma unroll
    for (int i = 0; i < 8; ++i) d = fmaf(w8[i], olat[64 * q + 8 * c8 + i], d);
  }
  d = lanes_sum<2>(d);
  if (q == 0) attn[static_cast<size_t>(b) * H * kV + h * kV + v] = static_cast<uint16_t>(f2bf(d));
}

// The same merge for at most 64 splits in one memory round trip: every load a
// thread needs -- the write slot, split (lane)'s max and sum, its latent column
// of every split's output, its row quarter of W_UV -- is issued at the start,
// none behind a branch (splits past the write slot are allocated and read but
// weighted zero). The max is a wave reduction over the lanes' splits; each
// split's weight reaches the other lanes by readlane, and the denominator and
// the weighted sum run in split order as in the loop form.
constexpr int kFastMergeSplits = 64;
// One block per (head, sequence), every load issued first and 16 bytes wide:
// thread t takes latent columns 8 (t % 32) .. + 7 of splits t / 32, t / 32 + 8,
// ... (NSP / 8 loads), weights them with w_s = l_s e^(m_s - M), and the eight
// split groups meet -- lane pairs (l, l ^ 32) in registers, then the four
// waves in order through LDS -- in o_lat = sum_s w_s op_s / sum_s w_s (f32).
// Then attn[b, h*64 + v] = bf16(W_UV[h][v] . o_lat).
// Each (head, sequence) takes VP blocks, each merging the splits (the cheap part,
// done by all VP) and applying W_UV for its 64 / VP value rows: smaller blocks,
// two of which share a CU and overlap their round trips (VP = 2: MLA core at
// 8 x 8192 17.8-18.1 -> 17.4-17.9 us, MiniCPM3 bs=1 369 -> 373 tok/s; VP = 4 was
// slower at batch 8).
constexpr int kMergeParts = 2;
template <int NSP, int VP>   // splits, rounded up to 16 / 32 / 64; blocks per head's value rows
__global__ __launch_bounds__(kThreads) void mla_combine_up_fast_kernel(
    const uint16_t* __restrict__ op, const float* __restrict__ mp, const float* __restrict__ lp,
    const int* __restrict__ wr, int ns, int split, int H, int cap, const uint16_t* __restrict__ w_kv_b,
    uint16_t* __restrict__ attn) {
  static_assert(NSP % 8 == 0 && NSP <= kWave, "splits in eight groups, one lane each for the weights");
  constexpr int kPer = NSP / 8;   // splits per thread
  constexpr int kVR = kV / VP;    // value rows of this block
  constexpr int kTPR = kThreads / kVR;   // threads per value row
  constexpr int kCPT = kLat / kTPR;      // latent columns per thread
  __shared__ float red[kWaves][kLat];
  __shared__ float olat[kLat];
  const int h = blockIdx.x / VP;
  const int vpart = blockIdx.x % VP;
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(t / kWave);
  const size_t srow = static_cast<size_t>(b) * ns * H + h;   // (b, s=0, h)
  // 1. every load, none behind a branch (a split past ns re-reads split ns - 1)
  const int last_raw = wr[b];
  const int sl = min(lane, ns - 1);
  const float m_l = mp[srow + static_cast<size_t>(sl) * H];
  const float l_l = lp[srow + static_cast<size_t>(sl) * H];
  const int cc = lane & 31;               // columns 8cc .. 8cc + 7
  const int hi = lane >> 5;
  const int sg = 2 * wv + hi;             // splits sg + 8i
  uint4 ov[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    ov[i] = ld16(op + (srow + static_cast<size_t>(min(sg + 8 * i, ns - 1)) * H) * kLat + 8 * cc);
  const int v = vpart * kVR + t / kTPR, q = t % kTPR;   // value row v, latent slice q
  const uint16_t* wrow = w_kv_b + (static_cast<size_t>(h) * kKvB + kNope + v) * kLat + kCPT * q;
  uint4 wv8[kCPT / 8];
#pragma unroll
  for (int c8 = 0; c8 < kCPT / 8; ++c8) wv8[c8] = ld16(wrow + 8 * c8);
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the first is read
  // 2. weights of the live splits (lane s holds split s)
  const int last = last_raw < 0 ? 0 : (last_raw >= cap ? cap - 1 : last_raw);
  const int nsa = min(ns, last / split + 1);
  const bool live = lane < nsa;
  const float M = lanes_max<6>(live ? m_l : -INFINITY);
  const float w = live ? l_l * expf(m_l - M) : 0.f;
  const float L = lanes_sum<6>(w);
  // 3. this thread's splits in order (dead splits add exact zeros: their weight
  //    and their value are selected away), then the lane pair, then the waves
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const float w_lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), 2 * wv + 8 * i));
    const float w_hi =
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), 2 * wv + 1 + 8 * i));
    const float ws = hi ? w_hi : w_lo;
    const bool in = sg + 8 * i < nsa;
    float x[8];
    unpack8(ov[i], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = fmaf(ws, in ? x[j] : 0.f, acc[j]);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[j]), __float_as_uint(acc[j]), false, false);
    acc[j] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  }
  if (hi == 0) {
    *reinterpret_cast<float4*>(&red[wv][8 * cc]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4*>(&red[wv][8 * cc + 4]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  lds_barrier();
  olat[t] = (((red[0][t] + red[1][t]) + red[2][t]) + red[3][t]) / L;
  lds_barrier();
  // 4. attn[b, h*64 + v] = bf16(W_UV[h][v] . o_lat)
  float d = 0.f;
#pragma unroll
  for (int c8 = 0; c8 < kCPT / 8; ++c8) {
    float w8[8];
    unpack8(wv8[c8], w8);
#pragma unroll
    for (int i = 0; i < 8; ++i) d = fmaf(w8[i], olat[kCPT * q + 8 * c8 + i], d);
  }
  d = lanes_sum<log2_const(kTPR)>(d);
  if (q == 0) attn[static_cast<size_t>(b) * H * kV + h * kV + v] = static_cast<uint16_t>(f2bf(d));
}

// ------------------------------------------------------------- rows_residual
// out[m, i] = bf16(res[m, i] + bf16(bf16(sum_s part[s, m, i]) * alpha)), 8 elements
// per thread.
template <int KS>   // the split count: exactly the live partials are loaded
__global__ __launch_bounds__(kThreads) void rows_residual_kernel(
    const float* __restrict__ part, const uint16_t* __restrict__ res, float alpha,
    uint16_t* __restrict__ out, int M, int N) {
  const size_t e0 = (static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x) * 8;
  const size_t total = static_cast<size_t>(M) * N;
  if (e0 >= total) return;
  const uint4 rv = ld16(res + e0);   // issued with the partials: one round trip
  float acc[8];
  sum_splits8<KS>(part + e0, total, KS, acc);
  float r[8];
  unpack8(rv, r);
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = round_bf(r[i] + round_bf(round_bf(acc[i]) * alpha));
  st16(out + e0, pack8(o));
}


// --------------------------------------------------------------- rope_attend
// MiniCPM3 decode attention over the assembled per-head cache Hugging Face
// keeps (k [cap, heads, nope + rope], v [cap, heads, v_dim]): the non-absorbed
// form, in the order of examples/minicpm3_4b-cutedsl/kernels/reference_ops.py:87-130.
// The query's rotary slice is rotated at pos (each product and the sum landing
// in bf16), the whole query is multiplied by the bf16 scale in bf16, scores are
// f32 dots, the softmax weights stay f32 into the value sum, and the token's own
// key and value join the context through a log-sum-exp merge.
//   rope_attend_split  per (split of 256 context rows, head): the split's max,
//                      sum and unnormalised weighted values; splits past ctx
//                      exit at once.
//   rope_attend_merge  per head: the token's key [k_nope | rotated k_rope] and
//                      value (to k_new / v_new), its score, and the merge of the
//                      live splits into bf16 attn.
constexpr int kRaSplit = 256;
constexpr int kRaMaxQK = 256;
constexpr int kRaMaxV = 128;

struct RopeAttendArgs {
  const uint16_t* q_up;    // [heads, qk]: [q_nope | q_rope] (rotary slice unrotated)
  const uint16_t* kv_up;   // [heads, nope + v_dim]: [k_nope | v]
  const uint16_t* k_rope;  // [rope] unrotated shared rotary key
  const uint16_t* cos_t;   // [rope_rows, rope]
  const uint16_t* sin_t;
  int rope_rows;
  const int* pos;          // [1] rotary position
  const uint16_t* kc;      // [cap, heads, qk]
  const uint16_t* vc;      // [cap, heads, v_dim]
  const int* ctx;          // [1] context rows held by the cache
  const uint16_t* scale;   // [1] bf16
  int cap, heads, nope, rope, vd;
  float* op;               // [ns, heads, v_dim]
  float* mp;               // [ns, heads]
  float* lp;               // [ns, heads]
  uint16_t* attn;          // [heads * v_dim]
  uint16_t* k_new;         // [heads * qk], optional
  uint16_t* v_new;         // [heads * v_dim], optional
  int* err;
};

// Rotate-half of a `rope`-wide slice x at index j, each product and the sum in bf16.
TFA_DEV float rope_bf(const uint16_t* x, int j, int half, float c, float s) {
  const float xv = bf2f(x[j]);
  const float r = j < half ? -bf2f(x[j + half]) : bf2f(x[j - half]);
  return round_bf(round_bf(xv * c) + round_bf(r * s));
}

TFA_DEV int ra_pos(const RopeAttendArgs& a) {
  const int p = a.pos[0];
  return (p < 0 || p >= a.rope_rows) ? 0 : p;
}

TFA_DEV int ra_ctx(const RopeAttendArgs& a) {
  const int n = a.ctx[0];
  return n < 0 ? 0 : (n > a.cap ? a.cap : n);
}

// qs[d] = bf16(query[d] * scale) for head h, the rotary slice rotated at p.
TFA_DEV void ra_query(const RopeAttendArgs& a, int h, int p, float* qs) {
  const int qk = a.nope + a.rope;
  const uint16_t* q = a.q_up + static_cast<size_t>(h) * qk;
  const float sc = bf2f(a.scale[0]);
  const size_t pr = static_cast<size_t>(p) * a.rope;
  for (int d = threadIdx.x; d < qk; d += blockDim.x) {
    float v;
    if (d < a.nope) {
      v = bf2f(q[d]);
    } else {
      const int j = d - a.nope;
      v = rope_bf(q + a.nope, j, a.rope / 2, bf2f(a.cos_t[pr + j]), bf2f(a.sin_t[pr + j]));
    }
    qs[d] = round_bf(v * sc);
  }
}

__global__ __launch_bounds__(kThreads) void rope_attend_split_kernel(const RopeAttendArgs a) {
  __shared__ float qs[kRaMaxQK];
  __shared__ float ps[kRaSplit];
  __shared__ float red[2][kWaves];
  __shared__ float ov[kWaves][kRaMaxV];
  const int s = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
  const int lane = t & (kWave - 1), wid = t / kWave;
  const int n = ra_ctx(a);
  const int start = s * kRaSplit;
  if (start >= n) return;  // whole block
  const int len = min(n - start, kRaSplit);
  ra_query(a, h, ra_pos(a), qs);
  lds_barrier();

  // scores: one context row per thread
  const int qk = a.nope + a.rope;
  float sco = -INFINITY;
  if (t < len) {
    const uint16_t* krow = a.kc + (static_cast<size_t>(start + t) * a.heads + h) * qk;
    float acc = 0.f;
    for (int c = 0; c < qk; c += 8) {
      float f[8];
      unpack8(ld16(krow + c), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fmaf(qs[c + i], f[i], acc);
    }
    sco = acc;
  }
  float m = wave_max(sco);
  if (lane == 0) red[0][wid] = m;
  lds_barrier();
  m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float e = t < len ? expf(sco - m) : 0.f;
  ps[t] = e;
  const float l = wave_sum(e);
  if (lane == 0) red[1][wid] = l;
  lds_barrier();

  // weighted values: wave w takes rows 64w .. 64w+63 of the split, lanes the value dims
  float acc0 = 0.f, acc1 = 0.f;
  const int j1 = min(len, (wid + 1) * kWave);
  for (int j = wid * kWave; j < j1; ++j) {
    const uint16_t* vrow = a.vc + (static_cast<size_t>(start + j) * a.heads + h) * a.vd;
    const float pj = ps[j];
    if (lane < a.vd) acc0 = fmaf(pj, bf2f(vrow[lane]), acc0);
    if (lane + kWave < a.vd) acc1 = fmaf(pj, bf2f(vrow[lane + kWave]), acc1);
  }
  ov[wid][lane] = acc0;
  ov[wid][lane + kWave] = acc1;
  lds_barrier();
  for (int d = t; d < a.vd; d += kThreads)
    a.op[(static_cast<size_t>(s) * a.heads + h) * a.vd + d] = (ov[0][d] + ov[1][d]) + (ov[2][d] + ov[3][d]);
  if (t == 0) {
    a.mp[s * a.heads + h] = m;
    a.lp[s * a.heads + h] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  }
}

__global__ __launch_bounds__(kThreads) void rope_attend_merge_kernel(const RopeAttendArgs a) {
  __shared__ float qs[kRaMaxQK];
  __shared__ float kn[kRaMaxQK];
  __shared__ float scr[kWaves];
  const int h = blockIdx.x, t = threadIdx.x;
  const int qk = a.nope + a.rope, kvw = a.nope + a.vd;
  if (h == 0 && t == 0) {
    const int p = a.pos[0], n = a.ctx[0];
    if (p < 0 || p >= a.rope_rows) set_err(a.err, 5);
    if (n < 0 || n > a.cap) set_err(a.err, 4);
  }
  const int p = ra_pos(a);
  const int n = ra_ctx(a);
  ra_query(a, h, p, qs);
  const uint16_t* kv = a.kv_up + static_cast<size_t>(h) * kvw;
  const size_t pr = static_cast<size_t>(p) * a.rope;
  for (int d = t; d < qk; d += kThreads) {
    float v;
    if (d < a.nope) {
      v = bf2f(kv[d]);
    } else {
      const int j = d - a.nope;
      v = rope_bf(a.k_rope, j, a.rope / 2, bf2f(a.cos_t[pr + j]), bf2f(a.sin_t[pr + j]));
    }
    kn[d] = v;
    if (a.k_new) a.k_new[static_cast<size_t>(h) * qk + d] = static_cast<uint16_t>(f2bf(v));
  }
  if (a.v_new)
    for (int d = t; d < a.vd; d += kThreads) a.v_new[static_cast<size_t>(h) * a.vd + d] = kv[a.nope + d];
  lds_barrier();
  float part = 0.f;
  for (int d = t; d < qk; d += kThreads) part = fmaf(qs[d], kn[d], part);
  const float snew = block_sum(part, scr);

  const int nact = (n + kRaSplit - 1) / kRaSplit;
  float peak = snew;
  for (int j = 0; j < nact; ++j) peak = fmaxf(peak, a.mp[j * a.heads + h]);
  const float enew = expf(snew - peak);
  float tot = enew;
  for (int j = 0; j < nact; ++j) tot = fmaf(a.lp[j * a.heads + h], expf(a.mp[j * a.heads + h] - peak), tot);
  for (int d = t; d < a.vd; d += kThreads) {
    float w = enew * bf2f(kv[a.nope + d]);
    for (int j = 0; j < nact; ++j)
      w = fmaf(a.op[(static_cast<size_t>(j) * a.heads + h) * a.vd + d], expf(a.mp[j * a.heads + h] - peak), w);
    a.attn[static_cast<size_t>(h) * a.vd + d] = static_cast<uint16_t>(f2bf(w / tot));
  }
}

}  // namespace

// ------------------------------------------------- no-allocation rope_attend
// tfa_rope_attend_noalloc keeps the split partials (op [ns, heads, v_dim], then
// mp and lp [ns, heads]) in this array instead of a caller's workspace. Each GPU
// the library runs on holds its own copy until the process ends. In host code
// the name is only a stand-in: the device address comes from
// hipGetSymbolAddress, once per device, and only that address reaches a kernel.
constexpr int64_t kRaScratchFloats = int64_t(1) << 20;   // 4 MiB
static __device__ __align__(256) float scratch[kRaScratchFloats];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_base[kMaxScratchDevices] = {};

// The current device's address of `scratch`, resolved on its first use there.
int scratch_base(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TFA_ERR_LAUNCH, "tfa_rope_attend_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(TFA_ERR_ARG, "tfa_rope_attend_noalloc: device %d beyond the %d the library tracks", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_base[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(TFA_ERR_LAUNCH, "tfa_rope_attend_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_base[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_base[dev];
  return TFA_OK;
}

}  // namespace

extern "C" {

int tfa_mla_prep(const float* part, int64_t ks, int64_t batch, int64_t q_lora, const void* gamma_q_a,
                 const void* gamma_kv_a, float eps, const void* cos_t, const void* sin_t,
                 int64_t rope_rows, const int* pos, void* latent_cache, void* rope_cache, int64_t cap,
                 void* q_n, int* err, hipStream_t stream) {
  TFA_NONNULL(part);
  TFA_NONNULL(gamma_q_a);
  TFA_NONNULL(gamma_kv_a);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  TFA_NONNULL(pos);
  TFA_NONNULL(latent_cache);
  TFA_NONNULL(rope_cache);
  TFA_NONNULL(q_n);
  TFA_REQUIRE(batch >= 1 && batch <= 65535, TFA_ERR_SHAPE, "tfa_mla_prep: batch %lld out of range", (long long)batch);
  TFA_REQUIRE(ks >= 1 && ks <= kMaxSplitsK, TFA_ERR_SHAPE, "tfa_mla_prep: ks %lld not in [1, %d]", (long long)ks, kMaxSplitsK);
  TFA_REQUIRE(q_lora >= 1 && q_lora <= 4 * kThreads, TFA_ERR_SHAPE,
              "tfa_mla_prep: q_lora %lld not in [1, %d]", (long long)q_lora, 4 * kThreads);
  TFA_REQUIRE(cap >= 1 && rope_rows >= 1, TFA_ERR_SHAPE, "tfa_mla_prep: empty cache or rope table");
  auto prep = [&](auto kc) {
    mla_prep_kernel<decltype(kc)::value><<<(int)batch, kThreads, 0, stream>>>(
        part, (int)ks, (int)batch, (int)q_lora, static_cast<const uint16_t*>(gamma_q_a),
        static_cast<const uint16_t*>(gamma_kv_a), eps, static_cast<const uint16_t*>(cos_t),
        static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos, static_cast<uint16_t*>(latent_cache),
        static_cast<uint16_t*>(rope_cache), (int)cap, static_cast<uint16_t*>(q_n), err);
  };
  static_assert(kMaxSplitsK == 8, "one instance per split count");
  switch (ks) {
    case 1: prep(std::integral_constant<int, 1>{}); break;
    case 2: prep(std::integral_constant<int, 2>{}); break;
    case 3: prep(std::integral_constant<int, 3>{}); break;
    case 4: prep(std::integral_constant<int, 4>{}); break;
    case 5: prep(std::integral_constant<int, 5>{}); break;
    case 6: prep(std::integral_constant<int, 6>{}); break;
    case 7: prep(std::integral_constant<int, 7>{}); break;
    default: prep(std::integral_constant<int, 8>{}); break;
  }
  return launched("mla_prep");
}

int tfa_mla_q_absorb(const float* q_part, int64_t ks, int64_t batch, int64_t heads, const void* w_kv_b,
                     const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos, void* q_abs,
                     int* err, hipStream_t stream) {
  TFA_NONNULL(q_part);
  TFA_NONNULL(w_kv_b);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  TFA_NONNULL(pos);
  TFA_NONNULL(q_abs);
  TFA_REQUIRE(batch >= 1 && batch <= kMaxBatch, TFA_ERR_SHAPE, "tfa_mla_q_absorb: batch %lld not in [1, %d]",
              (long long)batch, kMaxBatch);
  TFA_REQUIRE(heads >= 1 && heads <= kHeadRows, TFA_ERR_SHAPE, "tfa_mla_q_absorb: heads %lld not in [1, %d]",
              (long long)heads, kHeadRows);
  TFA_REQUIRE(ks >= 1 && ks <= kMaxSplitsK && rope_rows >= 1, TFA_ERR_SHAPE,
              "tfa_mla_q_absorb: ks %lld not in [1, %d] or empty rope table", (long long)ks, kMaxSplitsK);
  TFA_ALIGN16(q_part);
  TFA_ALIGN16(w_kv_b);
  if (batch == 1)
    mla_q_absorb_kernel<1><<<(int)heads, kThreads, 0, stream>>>(
        q_part, (int)ks, (int)batch, (int)heads, static_cast<const uint16_t*>(w_kv_b),
        static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos,
        static_cast<uint16_t*>(q_abs), err);
  else if (batch <= 8)
    mla_q_absorb_kernel<8><<<(int)heads, kThreads, 0, stream>>>(
        q_part, (int)ks, (int)batch, (int)heads, static_cast<const uint16_t*>(w_kv_b),
        static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos,
        static_cast<uint16_t*>(q_abs), err);
  else
    mla_q_absorb_kernel<kMaxBatch><<<(int)heads, kThreads, 0, stream>>>(
        q_part, (int)ks, (int)batch, (int)heads, static_cast<const uint16_t*>(w_kv_b),
        static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos,
        static_cast<uint16_t*>(q_abs), err);
  return launched("mla_q_absorb");
}

int tfa_mla_qb_absorb(const void* q_n, int64_t batch, int64_t heads, int64_t q_lora, const void* w_q_b,
                      const void* w_kv_b, const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos,
                      void* q_abs, int* err, hipStream_t stream) {
  TFA_NONNULL(q_n);
  TFA_NONNULL(w_q_b);
  TFA_NONNULL(w_kv_b);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  TFA_NONNULL(pos);
  TFA_NONNULL(q_abs);
  TFA_REQUIRE(batch >= 1 && batch <= kMaxBatch, TFA_ERR_SHAPE, "tfa_mla_qb_absorb: batch %lld not in [1, %d]",
              (long long)batch, kMaxBatch);
  TFA_REQUIRE(heads >= 1 && heads <= kHeadRows, TFA_ERR_SHAPE, "tfa_mla_qb_absorb: heads %lld not in [1, %d]",
              (long long)heads, kHeadRows);
  TFA_REQUIRE(q_lora == kQLora && rope_rows >= 1, TFA_ERR_SHAPE,
              "tfa_mla_qb_absorb: q_lora %lld (built for %d) or empty rope table", (long long)q_lora, kQLora);
  TFA_ALIGN16(q_n);
  TFA_ALIGN16(w_q_b);
  TFA_ALIGN16(w_kv_b);
  QbArgs a{};
  a.q_n = static_cast<const uint16_t*>(q_n);
  a.w_q_b = static_cast<const uint16_t*>(w_q_b);
  a.w_kv_b = static_cast<const uint16_t*>(w_kv_b);
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.rope_rows = (int)rope_rows;
  a.pos = pos;
  a.q_abs = static_cast<uint16_t*>(q_abs);
  a.err = err;
  a.B = (int)batch;
  a.H = (int)heads;
  const dim3 grid((unsigned)heads, 2);
  if (batch <= 16)
    mla_qb_absorb_kernel<1, false><<<grid, kThreads, 0, stream>>>(a);
  else
    mla_qb_absorb_kernel<2, false><<<grid, kThreads, 0, stream>>>(a);
  return launched("mla_qb_absorb");
}

int tfa_mla_prep_qb_absorb(const float* part, int64_t q_lora, const void* gamma_q_a, const void* gamma_kv_a,
                           float eps, const void* cos_t, const void* sin_t, int64_t rope_rows, const int* pos,
                           void* latent_cache, void* rope_cache, int64_t cap, const void* w_q_b, const void* w_kv_b,
                           int64_t heads, void* q_abs, int* err, hipStream_t stream) {
  TFA_NONNULL(part);
  TFA_NONNULL(gamma_q_a);
  TFA_NONNULL(gamma_kv_a);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  TFA_NONNULL(pos);
  TFA_NONNULL(latent_cache);
  TFA_NONNULL(rope_cache);
  TFA_NONNULL(w_q_b);
  TFA_NONNULL(w_kv_b);
  TFA_NONNULL(q_abs);
  TFA_REQUIRE(heads >= 1 && heads <= kHeadRows, TFA_ERR_SHAPE, "tfa_mla_prep_qb_absorb: heads %lld not in [1, %d]",
              (long long)heads, kHeadRows);
  TFA_REQUIRE(q_lora == kQLora && rope_rows >= 1 && cap >= 1, TFA_ERR_SHAPE,
              "tfa_mla_prep_qb_absorb: q_lora %lld (built for %d), empty rope table or cache", (long long)q_lora,
              kQLora);
  TFA_ALIGN16(part);
  TFA_ALIGN16(gamma_q_a);
  TFA_ALIGN16(w_q_b);
  TFA_ALIGN16(w_kv_b);
  QbArgs a{};
  a.part = part;
  a.gamma_q_a = static_cast<const uint16_t*>(gamma_q_a);
  a.gamma_kv_a = static_cast<const uint16_t*>(gamma_kv_a);
  a.eps = eps;
  a.lat_cache = static_cast<uint16_t*>(latent_cache);
  a.rope_cache = static_cast<uint16_t*>(rope_cache);
  a.cap = (int)cap;
  a.w_q_b = static_cast<const uint16_t*>(w_q_b);
  a.w_kv_b = static_cast<const uint16_t*>(w_kv_b);
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.rope_rows = (int)rope_rows;
  a.pos = pos;
  a.q_abs = static_cast<uint16_t*>(q_abs);
  a.err = err;
  a.B = 1;
  a.H = (int)heads;
  mla_qb_absorb_kernel<1, true><<<dim3((unsigned)heads, 2), kThreads, 0, stream>>>(a);
  return launched("mla_prep_qb_absorb");
}

int tfa_mla_attention(const void* q_abs, const void* latent_cache, const void* rope_cache, const int* wr,
                      int64_t batch, int64_t heads, int64_t cap, int64_t split, float scale, void* op,
                      float* mp, float* lp, int* err, hipStream_t stream) {
  TFA_NONNULL(q_abs);
  TFA_NONNULL(latent_cache);
  TFA_NONNULL(rope_cache);
  TFA_NONNULL(wr);
  TFA_NONNULL(op);
  TFA_NONNULL(mp);
  TFA_NONNULL(lp);
  TFA_REQUIRE(batch >= 1 && batch <= 65535, TFA_ERR_SHAPE, "tfa_mla_attention: batch %lld out of range", (long long)batch);
  TFA_REQUIRE(heads >= 1 && heads <= kHeadRows, TFA_ERR_SHAPE, "tfa_mla_attention: heads %lld not in [1, %d]",
              (long long)heads, kHeadRows);
  const bool whole = split % kHStep == 0;   // whole 128-position steps
  TFA_REQUIRE(split >= 1 && split <= 8 * kHStep && (whole || (split % kWaveRows == 0 && split < kHStep)),
              TFA_ERR_SHAPE, "tfa_mla_attention: split %lld must be 32, 64, 96 or a multiple of 128 up to 1024",
              (long long)split);
  TFA_REQUIRE(cap >= 1 && cap % split == 0 && cap / split <= kMaxSplits, TFA_ERR_SHAPE,
              "tfa_mla_attention: cap %lld must be a multiple of split %lld with at most %d splits",
              (long long)cap, (long long)split, kMaxSplits);
  TFA_ALIGN16(q_abs);
  TFA_ALIGN16(latent_cache);
  TFA_ALIGN16(rope_cache);
  TFA_ALIGN16(op);
  MlaAttnArgs a{};
  a.q = static_cast<const uint16_t*>(q_abs);
  a.lat = static_cast<const uint16_t*>(latent_cache);
  a.rk = static_cast<const uint16_t*>(rope_cache);
  a.wr = wr;
  a.op = static_cast<uint16_t*>(op);
  a.mp = mp;
  a.lp = lp;
  a.err = err;
  a.H = (int)heads;
  a.cap = (int)cap;
  a.ns = (int)(cap / split);
  a.tiles = (int)(split / (whole ? kHStep : AttnShape<1>::step));
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid(a.ns, (unsigned)batch);
  if (whole)
    mla_attn_heads_kernel<<<grid, kHW * kWave, 0, stream>>>(a);
  else
    mla_attn_kernel<1><<<grid, 3 * 1 * kWave, 0, stream>>>(a);
  return launched("mla_attn");
}

int tfa_mla_combine_up(const void* op, const float* mp, const float* lp, const int* wr, int64_t splits,
                       int64_t split, int64_t batch, int64_t heads, int64_t cap, const void* w_kv_b,
                       void* attn, hipStream_t stream) {
  TFA_NONNULL(op);
  TFA_NONNULL(mp);
  TFA_NONNULL(lp);
  TFA_NONNULL(wr);
  TFA_NONNULL(w_kv_b);
  TFA_NONNULL(attn);
  TFA_REQUIRE(splits >= 1 && splits <= kMaxSplits && split >= 1 && splits * split == cap, TFA_ERR_SHAPE,
              "tfa_mla_combine_up: %lld splits of %lld do not tile cap %lld (at most %d splits)",
              (long long)splits, (long long)split, (long long)cap, kMaxSplits);
  TFA_REQUIRE(batch >= 1 && batch <= 65535 && heads >= 1 && heads <= kHeadRows, TFA_ERR_SHAPE,
              "tfa_mla_combine_up: batch %lld / heads %lld out of range", (long long)batch, (long long)heads);
  TFA_ALIGN16(op);
  TFA_ALIGN16(w_kv_b);
  auto fast = [&](auto nsp) {
    mla_combine_up_fast_kernel<decltype(nsp)::value, kMergeParts>
        <<<dim3((unsigned)(heads * kMergeParts), (unsigned)batch), kThreads, 0, stream>>>(
            static_cast<const uint16_t*>(op), mp, lp, wr, (int)splits, (int)split, (int)heads, (int)cap,
            static_cast<const uint16_t*>(w_kv_b), static_cast<uint16_t*>(attn));
  };
  if (splits <= 16)
    fast(std::integral_constant<int, 16>{});
  else if (splits <= 32)
    fast(std::integral_constant<int, 32>{});
  else if (splits <= kFastMergeSplits)
    fast(std::integral_constant<int, kFastMergeSplits>{});
  else
    mla_combine_up_kernel<<<dim3((unsigned)heads, (unsigned)batch), kThreads, 0, stream>>>(
        static_cast<const uint16_t*>(op), mp, lp, wr, (int)splits, (int)split, (int)heads, (int)cap,
        static_cast<const uint16_t*>(w_kv_b), static_cast<uint16_t*>(attn));
  return launched("mla_combine_up");
}

int tfa_rows_residual(const float* part, int64_t ks, const void* residual, float alpha, void* out,
                      int64_t m, int64_t n, hipStream_t stream) {
  TFA_NONNULL(part);
  TFA_NONNULL(residual);
  TFA_NONNULL(out);
  TFA_REQUIRE(ks >= 1 && ks <= kMaxSplitsK && m >= 1 && n >= 8 && n % 8 == 0, TFA_ERR_SHAPE,
              "tfa_rows_residual: need ks in [1, %d], m >= 1 and n a positive multiple of 8", kMaxSplitsK);
  TFA_ALIGN16(part);
  TFA_ALIGN16(residual);
  TFA_ALIGN16(out);
  const int64_t blocks = (m * n / 8 + kThreads - 1) / kThreads;
  auto run = [&](auto kc) {
    rows_residual_kernel<decltype(kc)::value><<<(unsigned)blocks, kThreads, 0, stream>>>(
        part, static_cast<const uint16_t*>(residual), alpha, static_cast<uint16_t*>(out), (int)m, (int)n);
  };
  switch (ks) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    case 4: run(std::integral_constant<int, 4>{}); break;
    case 5: run(std::integral_constant<int, 5>{}); break;
    case 6: run(std::integral_constant<int, 6>{}); break;
    case 7: run(std::integral_constant<int, 7>{}); break;
    default: run(std::integral_constant<int, 8>{}); break;
  }
  return launched("rows_residual");
}

int64_t tfa_rope_attend_splits(int64_t cap) { return cap <= 0 ? 0 : (cap + kRaSplit - 1) / kRaSplit; }

int tfa_rope_attend(const void* q_up, const void* kv_up, const void* k_rope, const void* cos_t,
                    const void* sin_t, int64_t rope_rows, const int* pos, const void* k_cache,
                    const void* v_cache, int64_t cap, const int* ctx, const void* scale,
                    int64_t heads, int64_t nope, int64_t rope, int64_t v_dim, float* op, float* mp,
                    float* lp, void* attn, void* k_new, void* v_new, int* err, hipStream_t stream) {
  TFA_NONNULL(q_up);
  TFA_NONNULL(kv_up);
  TFA_NONNULL(k_rope);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  TFA_NONNULL(pos);
  TFA_NONNULL(ctx);
  TFA_NONNULL(scale);
  TFA_NONNULL(attn);
  TFA_REQUIRE(heads >= 1 && heads <= 65535 && nope >= 0 && rope >= 2 && rope % 2 == 0 &&
                  (nope + rope) % 8 == 0 && nope + rope <= kRaMaxQK && v_dim >= 1 && v_dim <= kRaMaxV &&
                  rope_rows >= 1 && cap >= 0,
              TFA_ERR_SHAPE,
              "tfa_rope_attend: need heads >= 1, even rope, (nope + rope) a multiple of 8 up to %d, "
              "v_dim in [1, %d]", kRaMaxQK, kRaMaxV);
  RopeAttendArgs a{};
  a.q_up = static_cast<const uint16_t*>(q_up);
  a.kv_up = static_cast<const uint16_t*>(kv_up);
  a.k_rope = static_cast<const uint16_t*>(k_rope);
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.rope_rows = (int)rope_rows;
  a.pos = pos;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.ctx = ctx;
  a.scale = static_cast<const uint16_t*>(scale);
  a.cap = (int)cap;
  a.heads = (int)heads;
  a.nope = (int)nope;
  a.rope = (int)rope;
  a.vd = (int)v_dim;
  a.op = op;
  a.mp = mp;
  a.lp = lp;
  a.attn = static_cast<uint16_t*>(attn);
  a.k_new = static_cast<uint16_t*>(k_new);
  a.v_new = static_cast<uint16_t*>(v_new);
  a.err = err;
  const int64_t ns = tfa_rope_attend_splits(cap);
  if (ns > 0) {
    TFA_NONNULL(k_cache);
    TFA_NONNULL(v_cache);
    TFA_NONNULL(op);
    TFA_NONNULL(mp);
    TFA_NONNULL(lp);
    TFA_ALIGN16(k_cache);
    rope_attend_split_kernel<<<dim3((unsigned)ns, (unsigned)heads), kThreads, 0, stream>>>(a);
    const int st = launched("rope_attend_split");
    if (st != TFA_OK) return st;
  }
  rope_attend_merge_kernel<<<(unsigned)heads, kThreads, 0, stream>>>(a);
  return launched("rope_attend_merge");
}

int64_t tfa_rope_attend_noalloc_max_floats(void) { return kRaScratchFloats; }

int tfa_rope_attend_noalloc(const void* q_up, const void* kv_up, const void* k_rope, const void* cos_t,
                            const void* sin_t, int64_t rope_rows, const int* pos, const void* k_cache,
                            const void* v_cache, int64_t cap, const int* ctx, const void* scale,
                            int64_t heads, int64_t nope, int64_t rope, int64_t v_dim, void* attn,
                            void* k_new, void* v_new, int* err, hipStream_t stream) {
  float *op = nullptr, *mp = nullptr, *lp = nullptr;
  const int64_t ns = tfa_rope_attend_splits(cap);
  if (ns > 0) {
    TFA_REQUIRE(heads >= 1 && heads <= 65535 && v_dim >= 1 && v_dim <= kRaMaxV, TFA_ERR_SHAPE,
                "tfa_rope_attend_noalloc: need heads in [1, 65535] and v_dim in [1, %d]", kRaMaxV);
    const int64_t need = ns * heads * (v_dim + 2);
    TFA_REQUIRE(need <= kRaScratchFloats, TFA_ERR_CAPACITY,
                "tfa_rope_attend_noalloc: %lld splits x %lld heads x (v_dim %lld + 2) = %lld floats exceed the "
                "%lld-float scratch array; use tfa_rope_attend with a workspace",
                (long long)ns, (long long)heads, (long long)v_dim, (long long)need, (long long)kRaScratchFloats);
    float* base = nullptr;
    const int st = scratch_base(&base);
    if (st != TFA_OK) return st;
    op = base;
    mp = base + ns * heads * v_dim;
    lp = mp + ns * heads;
  }
  return tfa_rope_attend(q_up, kv_up, k_rope, cos_t, sin_t, rope_rows, pos, k_cache, v_cache, cap, ctx, scale,
                         heads, nope, rope, v_dim, op, mp, lp, attn, k_new, v_new, err, stream);
}

}  // extern "C"
