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
//   mla_attn      per (split of 64*tiles positions, sequence), bf16 MFMA:
//                 S = q_abs . [c | k_rope]^T, online softmax in f32, O += P . c;
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
constexpr int kTile = 64;      // positions per pipeline step
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

// ------------------------------------------------------------------ mla_prep
// One block per sequence. part: [ks, B, qa + 256 + 32] f32 split-K partials of
// x_n . [W_q_a; W_kv_a]^T.
__global__ __launch_bounds__(kThreads) void mla_prep_kernel(
    const float* __restrict__ part, int ks, int B, int qa, const uint16_t* __restrict__ gq,
    const uint16_t* __restrict__ gkv, float eps, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int rope_rows, const int* __restrict__ pos,
    uint16_t* __restrict__ lat_cache, uint16_t* __restrict__ rope_cache, int cap,
    uint16_t* __restrict__ q_n, int* err) {
  __shared__ float scratch[2][kWaves];
  __shared__ float kr[kRope];
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int row = qa + kLat + kRope;
  const size_t kstride = static_cast<size_t>(B) * row;
  const float* pb = part + static_cast<size_t>(b) * row;
  auto reduced = [&](int i) {
    return round_bf(sum_splits(pb + i, kstride, ks));   // the projection lands in bf16
  };

  // q_a -> LoRA norm
  float qv[4];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = t + kThreads * j;
    qv[j] = i < qa ? reduced(i) : 0.f;
    ss += qv[j] * qv[j];
  }
  // kv_c -> LoRA norm (the latent); the rope slice
  const float cv = reduced(qa + t);
  if (t < kRope) kr[t] = reduced(qa + kLat + t);
  const float rq = rsqrt_rn(block_sum(ss, scratch[0]) / static_cast<float>(qa) + eps);
  const float rk = rsqrt_rn(block_sum(cv * cv, scratch[1]) / static_cast<float>(kLat) + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = t + kThreads * j;
    if (i < qa)
      q_n[static_cast<size_t>(b) * qa + i] =
          static_cast<uint16_t>(f2bf(round_bf(qv[j] * rq) * bf2f(gq[i])));
  }
  const int p = pos[b];
  if (p < 0 || p >= cap || p >= rope_rows) {
    if (t == 0) set_err(err, 6);
    return;
  }
  lat_cache[(static_cast<size_t>(b) * cap + p) * kLat + t] =
      static_cast<uint16_t>(f2bf(round_bf(cv * rk) * bf2f(gkv[t])));
  if (t < kRope) {   // kr was written before the block sums' barriers
    const float x = kr[t];
    const float partner = t < kRope / 2 ? -kr[t + kRope / 2] : kr[t - kRope / 2];
    const float c = bf2f(cos_t[static_cast<size_t>(p) * kRope + t]);
    const float s = bf2f(sin_t[static_cast<size_t>(p) * kRope + t]);
    rope_cache[(static_cast<size_t>(b) * cap + p) * kRope + t] =
        static_cast<uint16_t>(f2bf(rope_bf(x, partner, c, s)));
  }
}

// -------------------------------------------------------------- mla_q_absorb
// One block per head; thread t owns latent column t. qpart: [ks, B, H*96] f32
// split-K partials of q_n . W_q_b^T. w_kv_b: [H*128, 256] (out, in).
__global__ __launch_bounds__(kThreads) void mla_q_absorb_kernel(
    const float* __restrict__ qpart, int ks, int B, int H, const uint16_t* __restrict__ w_kv_b,
    const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t, int rope_rows,
    const int* __restrict__ pos, uint16_t* __restrict__ q_abs, int* err) {
  __shared__ float qn[kMaxBatch][kNope];
  __shared__ float qr[kMaxBatch][kRope];
  const int h = blockIdx.x;
  const int t = threadIdx.x;
  const int qrow = H * (kNope + kRope);
  const size_t kstride = static_cast<size_t>(B) * qrow;
  // this head's W_UK column t, loaded while the partials are reduced
  float wc[kNope];
  const uint16_t* wuk = w_kv_b + static_cast<size_t>(h) * kKvB * kLat + t;
#pragma unroll
  for (int i = 0; i < kNope; ++i) wc[i] = bf2f(wuk[static_cast<size_t>(i) * kLat]);
  for (int e = t; e < B * (kNope + kRope); e += kThreads) {
    const int b = e / (kNope + kRope), i = e % (kNope + kRope);
    const float* src = qpart + static_cast<size_t>(b) * qrow + h * (kNope + kRope) + i;
    const float acc = sum_splits(src, kstride, ks);
    if (i < kNope) qn[b][i] = round_bf(acc);
    else qr[b][i - kNope] = round_bf(acc);
  }
  lds_barrier();
  for (int b = 0; b < B; ++b) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kNope; ++i) acc = fmaf(qn[b][i], wc[i], acc);
    q_abs[(static_cast<size_t>(b) * H + h) * kQK + t] = static_cast<uint16_t>(f2bf(acc));
  }
  for (int e = t; e < B * kRope; e += kThreads) {
    const int b = e / kRope, d = e % kRope;
    int p = pos[b];
    if (p < 0 || p >= rope_rows) {
      if (h == 0) set_err(err, 6);
      p = 0;
    }
    const float partner = d < kRope / 2 ? -qr[b][d + kRope / 2] : qr[b][d - kRope / 2];
    const float c = bf2f(cos_t[static_cast<size_t>(p) * kRope + d]);
    const float s = bf2f(sin_t[static_cast<size_t>(p) * kRope + d]);
    q_abs[(static_cast<size_t>(b) * H + h) * kQK + kLat + d] =
        static_cast<uint16_t>(f2bf(rope_bf(qr[b][d], partner, c, s)));
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
  int H, cap, ns, tiles;   // a split is `tiles` steps of 64 positions
  float scale;
  float scale_log2;   // scale * log2(e)
};

// LDS tiles keep a position per row. Latent rows are 512 bytes of 32 16-byte
// chunks, stored XOR-swizzled by the row: the score operand reads (16 rows, one
// chunk) and the transpose reads of the value product (8 rows x 32 bytes per
// half-wave) then both hit 16 distinct bank groups.
TFA_DEV int lat_slot(int row, int chunk) { return chunk ^ (((row & 7) << 1) | ((row >> 3) & 1)); }
TFA_DEV int rope_slot(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4
// of the 8-byte reads of lanes 4j + i / 4 (j = 0..3). Lane L reading row
// base + L / 4 at column col0 + 4 (L % 4) therefore receives
// C[base + j][col0 + i], j = 0..3 -- four consecutive positions of one latent
// column, the MFMA's K-major operand.
TFA_DEV uint2 ld_tr(const uint16_t* lds_elem) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_elem));
  return __builtin_bit_cast(uint2, v);
}

template <int D>   // tiles prefetched in registers
__global__ __launch_bounds__(kThreads) void mla_attn_kernel(const MlaAttnArgs a) {
  __shared__ uint4 lat_s[2][kTile][kLat / 8];
  __shared__ uint4 rope_s[2][kTile][kRope / 8];
  __shared__ __attribute__((aligned(16))) uint16_t p_s[kHeadRows][kTile + 4];
  __shared__ uint4 q_s[kHeadRows][kQK / 8 + 1];   // 592-byte rows: 16-row operand reads conflict-free
  __shared__ float red[kWaves][kHeadRows];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int t = threadIdx.x;
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const int s = blockIdx.x;
  const int b = blockIdx.y;

  int last = a.wr[b];
  if (last < 0 || last >= a.cap) {
    if (s == 0 && t == 0) set_err(a.err, 4);
    last = last < 0 ? -1 : a.cap - 1;
  }
  const int n = last + 1;
  const int split = kTile * a.tiles;
  const int pos0 = s * split;
  if (pos0 >= n) return;
  const int ntiles = min(a.tiles, (n - pos0 + kTile - 1) / kTile);
  const uint16_t* lat = a.lat + (static_cast<size_t>(b) * a.cap + pos0) * kLat;
  const uint16_t* rk = a.rk + (static_cast<size_t>(b) * a.cap + pos0) * kRope;

  // staging: thread t moves latent chunks (row 8i + t/32, chunk t%32), i < 8,
  // and rope chunk (row t/4, chunk t%4). Rows past the context are stored as
  // zero (stale slots may hold anything; their weight is zero).
  const int srow = t >> 5, schunk = t & 31;
  const int rrow = t >> 2, rchunk = t & 3;
  uint4 rl[D][8], rr[D];
  auto fetch = [&](int tile, uint4* dl, uint4& dr) __attribute__((always_inline)) {
    const uint16_t* lt = lat + static_cast<size_t>(tile) * kTile * kLat;
#pragma unroll
    for (int i = 0; i < 8; ++i) dl[i] = ld16_stream(lt + (8 * i + srow) * kLat + schunk * 8);
    dr = ld16_stream(rk + (static_cast<size_t>(tile) * kTile + rrow) * kRope + rchunk * 8);
  };
  auto keep = [](uint4 v, bool ok) __attribute__((always_inline)) {   // a value select, not an address select
    v.x = ok ? v.x : 0u;
    v.y = ok ? v.y : 0u;
    v.z = ok ? v.z : 0u;
    v.w = ok ? v.w : 0u;
    return v;
  };
  auto stage = [&](int tile, int buf, const uint4* dl, const uint4& dr) __attribute__((always_inline)) {
    const int base = pos0 + tile * kTile;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 8 * i + srow;
      lat_s[buf][row][lat_slot(row, schunk)] = keep(dl[i], base + row < n);
    }
    rope_s[buf][rrow][rope_slot(rrow, rchunk)] = keep(dr, base + rrow < n);
  };

  fetch(0, rl[0], rr[0]);
  // the query of all heads, resident in LDS (padding rows repeat the last head;
  // their results are never stored)
  {
    // every load first (one round trip), then the stores
    constexpr int kQChunks = kHeadRows * (kQK / 8);
    constexpr int kQPer = (kQChunks + kThreads - 1) / kThreads;
    uint4 qv[kQPer];
#pragma unroll
    for (int i = 0; i < kQPer; ++i) {
      const int e = min(t + i * kThreads, kQChunks - 1);
      const int h = e / (kQK / 8), c = e % (kQK / 8);
      qv[i] = ld16(a.q + (static_cast<size_t>(b) * a.H + min(h, a.H - 1)) * kQK + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < kQPer; ++i) {
      const int e = t + i * kThreads;
      if (e < kQChunks) q_s[e / (kQK / 8)][e % (kQK / 8)] = qv[i];
    }
  }
  stage(0, 0, rl[0], rr[0]);
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (1 + d < ntiles) fetch(1 + d, rl[d], rr[d]);

  // running state of the lane's head rows h = 16mt + 4g + r
  float m_run[3][4], l_run[3][4];
  f32x4 o_acc[3][4];   // [mt][nt]: rows 16mt + 4g + r, latent column 64 wid + 16 nt + n16
#pragma unroll
  for (int mt = 0; mt < 3; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m_run[mt][r] = -INFINITY;
      l_run[mt][r] = 0.f;
    }
#pragma unroll
  for (int mt = 0; mt < 3; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) o_acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int tt0 = 0; tt0 < ntiles; tt0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int tt = tt0 + j;
      if (tt >= ntiles) break;
      const int buf = tt & 1;
      lds_barrier();   // buf holds tile tt; every wave is done with buf ^ 1

      // scores of this wave's 16 positions against all heads
      const int prow = 16 * wid + n16;
      f32x4 sacc[3];
#pragma unroll
      for (int mt = 0; mt < 3; ++mt) sacc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 9; ++ks) {
        const uint4 bop = ks < 8 ? lat_s[buf][prow][lat_slot(prow, 4 * ks + g)]
                                 : rope_s[buf][prow][rope_slot(prow, g)];
#pragma unroll
        for (int mt = 0; mt < 3; ++mt)
          sacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(q_s[16 * mt + n16][4 * ks + g]), as_bf8(bop),
                                                             sacc[mt], 0, 0, 0);
      }
      // scores in log2 units (the scale folded in), their max over the wave's
      // 16 positions by DPP within each 16-lane row
      const bool valid = pos0 + tt * kTile + prow < n;
      float sv[3][4], mx[3][4];
#pragma unroll
      for (int mt = 0; mt < 3; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[mt][r] = valid ? sacc[mt][r] * a.scale_log2 : -INFINITY;
          mx[mt][r] = row16_max(sv[mt][r]);
        }
      if (n16 == 0) {
#pragma unroll
        for (int mt = 0; mt < 3; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[wid][16 * mt + 4 * g + r] = mx[mt][r];
      }
      lds_barrier();
      // online softmax: every wave forms the same tile max per head. The
      // running max (log2 units) is only raised -- and O rescaled -- when some
      // head's tile max passes it by more than kSlack, so the weights
      // exp2(s - m) stay <= 2^kSlack; every wave takes the same decision.
      float mtile[3][4];
      bool raise = false;
#pragma unroll
      for (int mt = 0; mt < 3; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int h = 16 * mt + 4 * g + r;
          mtile[mt][r] = fmaxf(fmaxf(red[0][h], red[1][h]), fmaxf(red[2][h], red[3][h]));
          raise |= mtile[mt][r] > m_run[mt][r] + kSlack;
        }
      if (__builtin_amdgcn_ballot_w64(raise) != 0) {
#pragma unroll
        for (int mt = 0; mt < 3; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float m_new = fmaxf(m_run[mt][r], mtile[mt][r]);
            const float alpha = m_run[mt][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[mt][r] - m_new);
            l_run[mt][r] *= alpha;
            m_run[mt][r] = m_new;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) o_acc[mt][nt][r] *= alpha;
          }
      }
#pragma unroll
      for (int mt = 0; mt < 3; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = __builtin_amdgcn_exp2f(sv[mt][r] - m_run[mt][r]);   // masked: exp2(-inf) = 0
          l_run[mt][r] += e;
          p_s[16 * mt + 4 * g + r][prow] = static_cast<uint16_t>(f2bf(e));   // bf16 weights into the value product
        }
      lds_barrier();

      // O[:, this wave's 64 latent columns] += P . C
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        uint4 aop[3];
#pragma unroll
        for (int mt = 0; mt < 3; ++mt) {
          const uint16_t* pr = &p_s[16 * mt + n16][32 * k2 + 4 * g];
          const uint2 lo = *reinterpret_cast<const uint2*>(pr);
          const uint2 hi = *reinterpret_cast<const uint2*>(pr + 16);
          aop[mt] = make_uint4(lo.x, lo.y, hi.x, hi.y);   // positions 32k2 + 4g + {0..3, 16..19}
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int col = 64 * wid + 16 * nt + 4 * (n16 & 3);
          const int r1 = 32 * k2 + 4 * g + (n16 >> 2);
          const int r2 = r1 + 16;
          const uint16_t* e1 = reinterpret_cast<const uint16_t*>(&lat_s[buf][r1][lat_slot(r1, col >> 3)]) + (col & 7);
          const uint16_t* e2 = reinterpret_cast<const uint16_t*>(&lat_s[buf][r2][lat_slot(r2, col >> 3)]) + (col & 7);
          const uint2 v1 = ld_tr(e1);
          const uint2 v2 = ld_tr(e2);
          const uint4 bop = make_uint4(v1.x, v1.y, v2.x, v2.y);
#pragma unroll
          for (int mt = 0; mt < 3; ++mt)
            o_acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(aop[mt]), as_bf8(bop), o_acc[mt][nt], 0, 0, 0);
        }
      }
      // tile tt + 1 (register slot j, loaded while this tile was computed) goes
      // to the other buffer, which every wave finished reading before this
      // tile's first barrier; the slot is refilled D tiles ahead
      if (tt + 1 < ntiles) {
        stage(tt + 1, buf ^ 1, rl[j], rr[j]);
        if (tt + 1 + D < ntiles) fetch(tt + 1 + D, rl[j], rr[j]);
      }
    }
  }

  // split sums: over the lane's 16 position columns, then over the waves
#pragma unroll
  for (int m = 1; m < 16; m <<= 1)
#pragma unroll
    for (int mt = 0; mt < 3; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) l_run[mt][r] += __shfl_xor(l_run[mt][r], m, kWave);
  if (n16 == 0) {
#pragma unroll
    for (int mt = 0; mt < 3; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wid][16 * mt + 4 * g + r] = l_run[mt][r];
  }
  lds_barrier();
  const size_t orow = (static_cast<size_t>(b) * a.ns + s) * a.H;
#pragma unroll
  for (int mt = 0; mt < 3; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 16 * mt + 4 * g + r;
      if (h >= a.H) continue;
      const float lt = (red[0][h] + red[1][h]) + (red[2][h] + red[3][h]);
      const float inv = 1.0f / lt;
      uint16_t* dst = a.op + (orow + h) * kLat + 64 * wid + n16;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) dst[16 * nt] = static_cast<uint16_t>(f2bf(o_acc[mt][nt][r] * inv));
      if (wid == 0 && n16 == 0) {
        a.mp[orow + h] = m_run[mt][r] * 0.6931471805599453f;   // natural-log units
        a.lp[orow + h] = lt;
      }
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
  __shared__ float scratch[kWaves];
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
  if ((t & (kWave - 1)) == 0) scratch[t / kWave] = mx;
  lds_barrier();
  const float M = fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
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
  d += __shfl_xor(d, 1, kWave);
  d += __shfl_xor(d, 2, kWave);
  if (q == 0) attn[static_cast<size_t>(b) * H * kV + h * kV + v] = static_cast<uint16_t>(f2bf(d));
}

// ------------------------------------------------------------- rows_residual
// out[m, i] = bf16(res[m, i] + bf16(bf16(sum_s part[s, m, i]) * alpha)), 8 elements
// per thread.
__global__ __launch_bounds__(kThreads) void rows_residual_kernel(
    const float* __restrict__ part, int ks, const uint16_t* __restrict__ res, float alpha,
    uint16_t* __restrict__ out, int M, int N) {
  const size_t e0 = (static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x) * 8;
  const size_t total = static_cast<size_t>(M) * N;
  if (e0 >= total) return;
  float acc[8];
  sum_splits8(part + e0, total, ks, acc);
  float r[8];
  unpack8(ld16(res + e0), r);
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
  mla_prep_kernel<<<(int)batch, kThreads, 0, stream>>>(
      part, (int)ks, (int)batch, (int)q_lora, static_cast<const uint16_t*>(gamma_q_a),
      static_cast<const uint16_t*>(gamma_kv_a), eps, static_cast<const uint16_t*>(cos_t),
      static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos, static_cast<uint16_t*>(latent_cache),
      static_cast<uint16_t*>(rope_cache), (int)cap, static_cast<uint16_t*>(q_n), err);
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
  TFA_ALIGN16(w_kv_b);
  mla_q_absorb_kernel<<<(int)heads, kThreads, 0, stream>>>(
      q_part, (int)ks, (int)batch, (int)heads, static_cast<const uint16_t*>(w_kv_b),
      static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos,
      static_cast<uint16_t*>(q_abs), err);
  return launched("mla_q_absorb");
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
  TFA_REQUIRE(split >= kTile && split % kTile == 0 && split <= 16 * kTile, TFA_ERR_SHAPE,
              "tfa_mla_attention: split %lld must be a multiple of %d, at most %d", (long long)split, kTile, 16 * kTile);
  TFA_REQUIRE(cap >= 1 && cap % split == 0 && cap / split <= kMaxSplits, TFA_ERR_SHAPE,
              "tfa_mla_attention: cap %lld must be a multiple of split %lld with at most %d splits",
              (long long)cap, (long long)split, kMaxSplits);
  TFA_ALIGN16(q_abs);
  TFA_ALIGN16(latent_cache);
  TFA_ALIGN16(rope_cache);
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
  a.tiles = (int)(split / kTile);
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid(a.ns, (unsigned)batch);
  mla_attn_kernel<2><<<grid, kThreads, 0, stream>>>(a);
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
  TFA_ALIGN16(w_kv_b);
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
  rows_residual_kernel<<<(unsigned)blocks, kThreads, 0, stream>>>(
      part, (int)ks, static_cast<const uint16_t*>(residual), alpha, static_cast<uint16_t*>(out), (int)m, (int)n);
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

}  // extern "C"
