// Split-KV GQA decode attention (head_dim 128) and the merge of its splits.
//
// attn_decode: one block per (split, kv head). The block scores its G query
// heads against the cached slots of its split that are <= wr (the newest slot),
// normalises against the split's own max in f32, lands the weights in bf16 and
// accumulates P.V in f32 -- the order of
// examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501 (attn_partial). Lanes:
// slot = lane / 16 picks one of four positions, dc = lane % 16 one 8-wide slice
// of D, so one load instruction of a wave reads four whole 256-byte key rows.
// Every K and V load of the split is issued before any arithmetic.
//
// Fused mode (q / k head scales given): the block starts from the raw q|k
// projection and applies the per-head Qwen3RMSNorm and the rotate-half RoPE at
// `pos` itself (the query of its G heads; the new key too in the one block whose
// split holds slot wr, which also writes that key into the cache). Each block
// redoes its two heads' norm from 512 bytes in L2 -- cheaper than any
// cross-block hand-off. Replaces examples/qwen3_1_7b-tilelang/fast/kernels.py:328-411
// (qk_rope_cache) in the step.
//
// attn_combine: log-sum-exp merge of the splits into bf16 head-major output,
// examples/qwen3_1_7b-tilelang/fast/kernels.py:504-540.
#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int D = 128;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;      // prepared q [hq*D]; fused mode: raw [q | k] [(hq+hkv)*D]
  const float* part;      // batched fused mode: q|k|v split-K partials [ks, B, (hq+2hkv)*D]
  int part_ks;
  size_t q_bstride;       // elements between sequences in q
  size_t cache_bstride;   // elements between sequences in k_cache / v_cache
  const uint16_t* gq;     // [D] q head scale (fused mode when non-null)
  const uint16_t* gk;     // [D] k head scale
  float eps_head;
  const uint16_t* cos_t;  // [mp_rows, D]
  const uint16_t* sin_t;
  int mp_rows;
  uint16_t* kc;           // [B, cap, hkv*D]
  uint16_t* vc;           // [B, cap, hkv*D]
  const int* pos;         // [B] rope position (fused mode)
  const int* wr;          // [B] newest slot; attend slots 0..wr
  float* op;              // [B, ns, hq, D]
  float* mp;              // [B, ns, hq]
  float* lp;              // [B, ns, hq]
  int neutral;            // write neutral partials for splits past the context
  uint16_t* out;          // attn_seq: bf16 output [B, hq*D]
  int* err;
  int hq, hkv, cap, ns;
  float scale;
};

TFA_DEV void set_err(int* err, int code) {
  if (err) atomicExch(err, code);
}

// Raw projection values of a 128-wide head for lane l: d = l and d = l + 64,
// landed in bf16 -- from a bf16 vector, or summed over split-K f32 partials.
TFA_DEV void head_raw(const uint16_t* raw, const float* part, int ks, size_t kstride, int lane,
                      float& x0, float& x1) {
  if (part) {
    x0 = round_bf(sum_splits(part + lane, kstride, ks));
    x1 = round_bf(sum_splits(part + lane + 64, kstride, ks));
  } else {
    x0 = bf2f(raw[lane]);
    x1 = bf2f(raw[lane + 64]);
  }
}

// The same values, loaded now and landed later: a kernel issues these loads,
// then its bulk loads, and only then lands them, so that its first wait covers
// every small load at once (vector loads complete in issue order). Nothing
// reads a loaded value before land(): a bf16 value stays in its 32-bit
// register as loaded, split-K partials are summed as sum_splits does.
template <bool PART>
struct HeadRaw {
  float v0[PART ? kMaxSplitsK : 1], v1[PART ? kMaxSplitsK : 1];
  uint32_t r0 = 0, r1 = 0;
  TFA_DEV void load(const uint16_t* raw, const float* part, int ks, size_t kstride, int lane) {
    if constexpr (PART) {
#pragma unroll
      for (int s = 0; s < kMaxSplitsK; ++s) {
        const size_t o = static_cast<size_t>(min(s, ks - 1)) * kstride;
        v0[s] = part[o + lane];
        v1[s] = part[o + lane + 64];
      }
    } else {
      r0 = raw[lane];
      r1 = raw[lane + 64];
    }
  }
  // The partials count as read here (an empty asm that takes and returns each),
  // so no part of their sum is moved up to the loads. (A bf16 value needs no
  // pin: nothing but its widening reads it.)
  TFA_DEV void pin() {
    if constexpr (PART) {
#pragma unroll
      for (int s = 0; s < kMaxSplitsK; ++s) asm volatile("" : "+v"(v0[s]), "+v"(v1[s]));
    }
  }
  TFA_DEV void land(int ks, float& x0, float& x1) {
    pin();
    if constexpr (PART) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int s = 0; s < kMaxSplitsK; ++s) {
        a0 += s < ks ? v0[s] : 0.f;
        a1 += s < ks ? v1[s] : 0.f;
      }
      x0 = round_bf(a0);
      x1 = round_bf(a1);
    } else {
      x0 = __uint_as_float(r0 << 16);
      x1 = __uint_as_float(r1 << 16);
    }
  }
};

// How the split attention gets its query: prepared (normed, rotated) bf16;
// fused from the raw [q | k] bf16 projection; fused from q|k|v split-K partials.
enum { QM_PREPARED = 0, QM_RAW = 1, QM_PART = 2 };

// Per-head Qwen3RMSNorm + rotate-half RoPE of one 128-wide head by one wave:
// lane l owns d = l and its rotation partner d = l + 64.
TFA_DEV void norm_rope_head_g(float x0, float x1, float g0, float g1, float eps, float c0, float s0,
                              float c1, float s1, float& o0, float& o1) {
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rs = rsqrt_rn(ss / static_cast<float>(D) + eps);
  const float n0 = round_bf(round_bf(x0 * rs) * g0);
  const float n1 = round_bf(round_bf(x1 * rs) * g1);
  // rotate_half: first half pairs with -x[d + 64], second half with +x[d - 64]
  o0 = round_bf(__fadd_rn(__fmul_rn(n0, c0), __fmul_rn(-n1, s0)));
  o1 = round_bf(__fadd_rn(__fmul_rn(n1, c1), __fmul_rn(n0, s1)));
}

TFA_DEV void norm_rope_head(float x0, float x1, const uint16_t* gam, float eps, float c0, float s0,
                            float c1, float s1, int lane, float& o0, float& o1) {
  norm_rope_head_g(x0, x1, bf2f(gam[lane]), bf2f(gam[lane + 64]), eps, c0, s0, c1, s1, o0, o1);
}

template <int G, int NIT, int QM>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(const AttnArgs a) {
  constexpr int SS = 16 * NIT;
  __shared__ float qs[G][D];
  __shared__ float knew[D];
  __shared__ float vnew[D];
  __shared__ float obuf[kWaves][G][D];
  __shared__ float red[2][kWaves][G];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int slot = lane >> 4;
  const int dc = lane & 15;
  // kv head fastest: the blocks of one split are dispatched together and read
  // the same cache rows (each position's row holds every kv head) close in time
  const int kvh = blockIdx.x;
  const int s = blockIdx.y;
  const int b = blockIdx.z;
  const int t = threadIdx.x;
  const int KN = a.hkv * D;
  uint16_t* kc = a.kc + b * a.cache_bstride;
  uint16_t* vc = a.vc + b * a.cache_bstride;
  float* op = a.op + static_cast<size_t>(b) * a.ns * a.hq * D;
  float* mp = a.mp + static_cast<size_t>(b) * a.ns * a.hq;
  float* lp = a.lp + static_cast<size_t>(b) * a.ns * a.hq;

  // 0. the loads that need nothing else, issued together: the write slot, the
  //    rope position and (fused mode) the raw head values of this wave's prologue
  //    items -- its query heads, the new key and (from partials) the new value,
  //    loaded whether or not this split turns out to hold the new slot -- or
  //    (prepared mode) the query. They complete in issue order, ahead of every
  //    K / V load, and are landed only after those are issued: the first wait
  //    covers them all, and the K / V loads go out one round trip after wr.
  constexpr bool fused = QM != QM_PREPARED;
  int last = a.wr[b];
  const int p_raw = fused ? a.pos[b] : 0;
  constexpr int kItems = (G + 2 + kWaves - 1) / kWaves;   // prologue items per wave: hh = wid + kWaves j
  constexpr int kQPer = (G * D + kThreads - 1) / kThreads; // prepared query values per thread
  const int rows = (a.hq + 2 * a.hkv) * D;   // q | k | v row width of the partials
  const uint16_t* qsrc = a.q ? a.q + b * a.q_bstride : nullptr;
  const float* psrc = a.part ? a.part + static_cast<size_t>(b) * rows : nullptr;
  const size_t kstride = static_cast<size_t>(rows) * gridDim.z;  // partials are [ks, B, rows]
  HeadRaw<QM == QM_PART> hr[kItems];
  uint32_t gr0[kItems], gr1[kItems];   // the item's norm scale (query: gamma_q, key: gamma_k)
  uint32_t qraw[kQPer];
  if constexpr (fused) {
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      // items past the value (and, without partials, the value itself: its row is
      // already in the cache) load the key's values, never used
      const int hh = min(wid + kWaves * j, QM == QM_PART ? G + 1 : G);
      const int off = hh < G ? (kvh * G + hh) * D : hh == G ? (a.hq + kvh) * D : (a.hq + a.hkv + kvh) * D;
      hr[j].load(QM == QM_RAW ? qsrc + off : nullptr, QM == QM_PART ? psrc + off : nullptr, a.part_ks, kstride, lane);
      const uint16_t* gam = hh < G ? a.gq : a.gk;
      gr0[j] = gam[lane];
      gr1[j] = gam[lane + 64];
    }
  } else {
#pragma unroll
    for (int u = 0; u < kQPer; ++u) qraw[u] = a.q[b * a.q_bstride + (kvh * G) * D + min(t + u * kThreads, G * D - 1)];
  }
  // a write slot outside the cache is flagged and clamped for the reads only:
  // no block then holds the new slot, so no cache row is written (attn_seq's rule)
  const bool wr_ok = last >= 0 && last < a.cap;
  if (!wr_ok) {
    if (s == 0 && kvh == 0 && t == 0) set_err(a.err, 4);
    last = last < 0 ? -1 : a.cap - 1;
  }
  const int n = last + 1;
  const int start = s * SS;
  if (start >= n) {
    if (a.neutral) {
      for (int e = t; e < G * D; e += kThreads) {
        const int g = e / D, d = e % D;
        const int h = kvh * G + g;
        op[(static_cast<size_t>(s) * a.hq + h) * D + d] = 0.f;
        if (d == 0) {
          mp[s * a.hq + h] = -1.0e30f;
          lp[s * a.hq + h] = 0.f;
        }
      }
    }
    return;
  }
  const bool has_new = fused && wr_ok && last < start + SS;  // this split holds the newest slot
  const bool new_v = has_new && QM == QM_PART;      // ... and also brings the new value row
  const int nwork = fused ? G + (has_new ? 1 : 0) + (new_v ? 1 : 0) : 0;

  // 1. the rope row (it needs the position), still ahead of the K / V
  int p = p_raw;
  if (fused && (p < 0 || p >= a.mp_rows)) {
    if (s == 0 && kvh == 0 && t == 0) set_err(a.err, 5);
    p = 0;
  }
  uint32_t cr0 = 0, sr0 = 0, cr1 = 0, sr1 = 0;
  if constexpr (fused) {
    cr0 = a.cos_t[static_cast<size_t>(p) * D + lane];
    sr0 = a.sin_t[static_cast<size_t>(p) * D + lane];
    cr1 = a.cos_t[static_cast<size_t>(p) * D + lane + 64];
    sr1 = a.sin_t[static_cast<size_t>(p) * D + lane + 64];
  }

  // 2. every K / V load of the split, unconditional: positions past the context
  //    read row n - 1 (in bounds) and are zeroed once landed, so no lane's load
  //    sits behind a branch and the first wait can count them all
  uint4 kv[NIT], vv[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int pi = min(start + it * 16 + wid * 4 + slot, n - 1);
    const size_t off = static_cast<size_t>(pi) * KN + kvh * D + 8 * dc;
    kv[it] = ld16_stream(kc + off);
    vv[it] = ld16_stream(vc + off);
  }

  // 3. land the small loads (nothing above this line waits for a load but wr)
  __builtin_amdgcn_sched_barrier(0);
  float x0[kItems], x1[kItems];
#pragma unroll
  for (int j = 0; j < kItems; ++j) hr[j].land(a.part_ks, x0[j], x1[j]);
  const float c0 = __uint_as_float(cr0 << 16), s0 = __uint_as_float(sr0 << 16);
  const float c1 = __uint_as_float(cr1 << 16), s1 = __uint_as_float(sr1 << 16);
  if constexpr (!fused) {
#pragma unroll
    for (int u = 0; u < kQPer; ++u) {
      const int e = t + u * kThreads;
      if (e < G * D) qs[e / D][e % D] = __uint_as_float(qraw[u] << 16);
    }
  }

  // the prologue's arithmetic while the K / V loads are in flight
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int hh = wid + kWaves * j;
    if (!fused || hh >= nwork) continue;
    float o0, o1;
    if (hh < G) {
      norm_rope_head_g(x0[j], x1[j], __uint_as_float(gr0[j] << 16), __uint_as_float(gr1[j] << 16), a.eps_head, c0,
                       s0, c1, s1, o0, o1);
      qs[hh][lane] = o0;
      qs[hh][lane + 64] = o1;
    } else if (hh == G) {
      norm_rope_head_g(x0[j], x1[j], __uint_as_float(gr0[j] << 16), __uint_as_float(gr1[j] << 16), a.eps_head, c0,
                       s0, c1, s1, o0, o1);
      knew[lane] = o0;
      knew[lane + 64] = o1;
      uint16_t* dst = kc + static_cast<size_t>(last) * KN + kvh * D;
      dst[lane] = static_cast<uint16_t>(f2bf(o0));
      dst[lane + 64] = static_cast<uint16_t>(f2bf(o1));
    } else {
      vnew[lane] = x0[j];
      vnew[lane + 64] = x1[j];
      uint16_t* dst = vc + static_cast<size_t>(last) * KN + kvh * D;
      dst[lane] = static_cast<uint16_t>(f2bf(x0[j]));
      dst[lane + 64] = static_cast<uint16_t>(f2bf(x1[j]));
    }
  }
  lds_barrier();

  // 3. scores (scale applied to the finished f32 dot), kept in registers: after
  //    the 16-lane DPP row sum every lane of a position's group holds its score.
  //    Reductions across the wave's four position slots use the gfx950 row
  //    swaps (no LDS round trip); the weights are exp2 of the scaled difference
  //    The query's values are bf16 (landed by the prep, or given so): packed in
  //    pairs, each score is four v_dot2 products of the raw key row.
  uint4 qp[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qp[g] = pack8(&qs[g][8 * dc]);
  float sv[G][NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int pi = start + it * 16 + wid * 4 + slot;
    const uint4 kr = (has_new && pi == last) ? pack8(&knew[8 * dc]) : kv[it];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = dot2_bf16(qp[g].x, kr.x, 0.f);
      d = dot2_bf16(qp[g].y, kr.y, d);
      d = dot2_bf16(qp[g].z, kr.z, d);
      d = dot2_bf16(qp[g].w, kr.w, d);
      d = row16_sum(d);
      sv[g][it] = pi < n ? d * a.scale : -INFINITY;
    }
  }

  // 4. the split's max and sum, f32: in-lane, across the wave's four position
  //    slots, then across the four waves through LDS
  float m[G], l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = sv[g][0];
#pragma unroll
    for (int it = 1; it < NIT; ++it) mx = fmaxf(mx, sv[g][it]);
    mx = rows4_max(mx);
    if (lane == 0) red[0][wid][g] = mx;
  }
  lds_barrier();
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = fmaxf(fmaxf(red[0][0][g], red[0][1][g]), fmaxf(red[0][2][g], red[0][3][g]));
    float ls = 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const float e = sv[g][it] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((sv[g][it] - m[g]) * kLog2e);
      ls += e;
      sv[g][it] = round_bf(e);  // bf16 weights into the value product
    }
    ls = rows4_sum(ls);
    if (lane == 0) red[1][wid][g] = ls;
  }

  // 5. P.V in registers
  float o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    float vf[8];
    const int pi = start + it * 16 + wid * 4 + slot;
    if (new_v && pi == last) {
#pragma unroll
      for (int i = 0; i < 8; ++i) vf[i] = vnew[8 * dc + i];
    } else {
      // a position past the context brought row n - 1: weight 0, value 0
      unpack8(pi < n ? vv[it] : make_uint4(0, 0, 0, 0), vf);
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) o[g][i] = fmaf(sv[g][it], vf[i], o[g][i]);
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o[g][i] = rows4_sum(o[g][i]);
    }
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) obuf[wid][g][8 * dc + i] = o[g][i];
  }
  lds_barrier();
#pragma unroll
  for (int g = 0; g < G; ++g)
    l[g] = (red[1][0][g] + red[1][1][g]) + (red[1][2][g] + red[1][3][g]);
  for (int e = t; e < G * D; e += kThreads) {
    const int g = e / D, d = e % D;
    const float v = (obuf[0][g][d] + obuf[1][g][d]) + (obuf[2][g][d] + obuf[3][g][d]);
    const int h = kvh * G + g;
    op[(static_cast<size_t>(s) * a.hq + h) * D + d] = v;
    if (d == 0) {
      mp[s * a.hq + h] = m[g];
      lp[s * a.hq + h] = l[g];
    }
  }
}

// attn_seq: the whole context of one (sequence, kv head) per block, with the
// query prep fused and no split merge -- for batches whose sequences x kv heads
// already fill the device (32 x 8 = 256 blocks, one per CU). The block sums its
// G query heads, its key head and its value head from the q|k|v split-K
// partials, applies the per-head norm and RoPE at pos[b], writes the new key
// and value rows to cache slot wr[b], and then streams its kv head's cache in
// two passes: keys -> every score of the context into LDS and the block max;
// values -> exp(s - max) in f32 summed for the denominator and landed in bf16
// into the f32 P.V. That is the order of the reference's unsplit softmax
// (exp against the row max, bf16 weights, one landing of o / l), with no
// per-split statistics. A position is one 256-byte cache row segment; lane
// (slot = l / 16, dc = l % 16) of wave w takes position 32 s + 4 w + slot of
// step s and the 8 dims 8 dc ..; the K steps then the V steps run through a
// ring of R 16-byte loads per lane, so the value loads are in flight while the
// last scores, the max and the weights are computed. Scores are v_dot2 bf16
// products of the raw key rows; the weights are computed lane-parallel over
// positions once the max is known and replace the scores in LDS. Replaces
// examples/qwen3_1_7b-tilelang/fast/kernels.py:328-411 (qk_rope_cache),
// :418-501 (attn_partial) and :504-540 (attn_combine) for one step.
// Score store: 128 KB of LDS, so a context of up to kSeqScores / G positions;
// it also keeps one block per CU (the blocks are as many as the CUs, and two on
// one CU would leave another idle for the whole launch).
constexpr int kSeqScores = 32768;
// Waves per block and 16-byte loads in flight per lane, measured at 32 x 8
// heads over 1000 / 2000 positions: 16 waves x 8 (four per SIMD, so one wave's
// dependent score / weight arithmetic hides under the others') 26.1 / 46.0 us,
// 8 x 16: 27.1 / 46.5, 8 x 32: 31.4 / 50.4, 12 x 16: 30.3 / 51.0. Four query
// heads per kv head need 8 waves to keep the per-wave output rows in LDS.
template <int G>
struct SeqShape {
  static constexpr int W = G <= 2 ? 16 : 8;
  static constexpr int R = G <= 2 ? 8 : 16;
  static constexpr int step = W * 4;   // positions per step (the score store's padding)
};

template <int G, int W = SeqShape<G>::W, int R = SeqShape<G>::R>
__global__ __launch_bounds__(W * kWave) void attn_seq_kernel(const AttnArgs a, uint16_t* __restrict__ out) {
  constexpr int kSeqThreads = W * kWave;
  constexpr int kSeqStep = W * 4;
  constexpr int kSeqRing = R;
  constexpr int kSeqWaves = W;
  __shared__ float sc[kSeqScores];   // [G][npos] scores of the context
  __shared__ float qs[G][D];
  __shared__ float knew[D];
  __shared__ float vnew[D];
  __shared__ float obuf[W][G][D];
  __shared__ float red[2][W][G];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int slot = lane >> 4;
  const int dc = lane & 15;
  const int kvh = blockIdx.x;
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  const int KN = a.hkv * D;
  uint16_t* kc = a.kc + b * a.cache_bstride;
  uint16_t* vc = a.vc + b * a.cache_bstride;
  uint16_t* ob = out + static_cast<size_t>(b) * a.hq * D + static_cast<size_t>(kvh) * G * D;

  // 1. the loads that need nothing else: the write slot, the rope position and
  //    the raw heads of the prologue (wave hh < G: query head kvh*G + hh; G: key;
  //    G+1: value); then, once the position is known, the rope row; then the
  //    first round of the cache stream. The raw heads and the rope row are landed
  //    only after that round is issued (loads complete in issue order).
  int last = a.wr[b];
  int p = a.pos[b];
  const int rows = (a.hq + 2 * a.hkv) * D;
  const size_t kstride = static_cast<size_t>(rows) * gridDim.y;   // partials are [ks, B, rows]
  const float* psrc = a.part + static_cast<size_t>(b) * rows;
  HeadRaw<true> hr;
  uint32_t gr0 = 0, gr1 = 0;   // the head's norm scale (query: gamma_q, key: gamma_k)
  if (wid < G + 2) {
    const int off = wid < G ? (kvh * G + wid) * D : wid == G ? (a.hq + kvh) * D : (a.hq + a.hkv + kvh) * D;
    hr.load(nullptr, psrc + off, a.part_ks, kstride, lane);
    const uint16_t* gam = wid < G ? a.gq : a.gk;
    gr0 = gam[lane];
    gr1 = gam[lane + 64];
  }
  if (last < 0 || last >= a.cap) {
    if (kvh == 0 && t == 0) set_err(a.err, 4);
    for (int e = t; e < G * D; e += kSeqThreads) ob[e] = 0;
    return;   // block-uniform: no barrier has been reached
  }
  if (p < 0 || p >= a.mp_rows) {
    if (kvh == 0 && t == 0) set_err(a.err, 5);
    p = 0;
  }
  const int n = last + 1;
  const int nst = (n + kSeqStep - 1) / kSeqStep;   // steps per pass
  const int npos = nst * kSeqStep;
  const int nch = 2 * nst;                         // K steps, then V steps
  const int pw = wid * 4 + slot;                   // this lane's position within a step
  const uint32_t cr0 = a.cos_t[static_cast<size_t>(p) * D + lane];
  const uint32_t sr0 = a.sin_t[static_cast<size_t>(p) * D + lane];
  const uint32_t cr1 = a.cos_t[static_cast<size_t>(p) * D + lane + 64];
  const uint32_t sr1 = a.sin_t[static_cast<size_t>(p) * D + lane + 64];

  // chunk c < nst: key step c; else value step c - nst. Positions past the
  // context read row n - 1 (in bounds) and are never used.
  auto chunk_ptr = [&](int c) -> const uint16_t* {
    const bool isv = c >= nst;
    const int pi = min((isv ? c - nst : c) * kSeqStep + pw, n - 1);
    return (isv ? vc : kc) + static_cast<size_t>(pi) * KN + kvh * D + 8 * dc;
  };
  uint4 ring[kSeqRing];
#pragma unroll
  for (int r = 0; r < kSeqRing; ++r) ring[r] = ld16_stream(chunk_ptr(min(r, nch - 1)));
  const float c0 = __uint_as_float(cr0 << 16), s0 = __uint_as_float(sr0 << 16);
  const float c1 = __uint_as_float(cr1 << 16), s1 = __uint_as_float(sr1 << 16);

  // 2. the prep's arithmetic while the first cache loads are in flight (the
  //    wave index is re-read through readfirstlane so that this branch and the
  //    loading one stay apart and the sums are not moved up to the loads)
  __builtin_amdgcn_sched_barrier(0);
  if (__builtin_amdgcn_readfirstlane(wid) < G + 2) {
    float x0, x1;
    hr.land(a.part_ks, x0, x1);
    asm volatile("" : "+v"(gr0), "+v"(gr1));
    if (wid <= G) {
      float o0, o1;
      norm_rope_head_g(x0, x1, __uint_as_float(gr0 << 16), __uint_as_float(gr1 << 16), a.eps_head, c0, s0, c1, s1,
                       o0, o1);
      if (wid < G) {
        qs[wid][lane] = o0;
        qs[wid][lane + 64] = o1;
      } else {
        knew[lane] = o0;
        knew[lane + 64] = o1;
        uint16_t* dst = kc + static_cast<size_t>(last) * KN + kvh * D;
        dst[lane] = static_cast<uint16_t>(f2bf(o0));
        dst[lane + 64] = static_cast<uint16_t>(f2bf(o1));
      }
    } else {
      vnew[lane] = x0;
      vnew[lane + 64] = x1;
      uint16_t* dst = vc + static_cast<size_t>(last) * KN + kvh * D;
      dst[lane] = static_cast<uint16_t>(f2bf(x0));
      dst[lane + 64] = static_cast<uint16_t>(f2bf(x1));
    }
  }
  lds_barrier();
  // the query as packed bf16 pairs (its values are bf16 already): scores are
  // v_dot2 products of the raw key rows, no unpacking
  uint32_t qp[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 q4 = pack8(&qs[g][8 * dc]);
    qp[g][0] = q4.x;
    qp[g][1] = q4.y;
    qp[g][2] = q4.z;
    qp[g][3] = q4.w;
  }
  const uint4 knp = pack8(&knew[8 * dc]);
  const uint4 vnp = pack8(&vnew[8 * dc]);
  const int clast = last / kSeqStep;   // the step holding the new slot

  float mloc[G], M[G], ls[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mloc[g] = -INFINITY;
    M[g] = 0.f;
    ls[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
  }

  // 3. the stream: scores (keys); then the block max and every weight of the
  //    wave's positions at once (lane-parallel over positions, not per row);
  //    then P.V (values). The chunk count is padded to whole ring rounds and
  //    every refill is issued (past the last chunk it re-reads that chunk;
  //    padding chunks are value steps past the context, weight 0), so the loop
  //    body is straight-line and each use waits only for its own load.
  const int nrounds = (nch + kSeqRing - 1) / kSeqRing;
  auto step = [&](const int c, uint4 v) __attribute__((always_inline)) {
    if (c < nst) {
      const int pi = c * kSeqStep + pw;
      if (c == clast && pi == last) v = knp;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = dot2_bf16(qp[g][0], v.x, 0.f);
        d = dot2_bf16(qp[g][1], v.y, d);
        d = dot2_bf16(qp[g][2], v.z, d);
        d = dot2_bf16(qp[g][3], v.w, d);
        d = row16_sum(d) * a.scale;
        if (pi < n) {
          mloc[g] = fmaxf(mloc[g], d);
          if (dc == 0) sc[g * npos + pi] = d;
        }
      }
      if (c == nst - 1) {   // every score is in: the block max, then the weights
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float mx = rows4_max(mloc[g]);
          if (lane == 0) red[0][wid][g] = mx;
        }
        lds_barrier();
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float mx = red[0][0][g];
#pragma unroll
          for (int w = 1; w < kSeqWaves; ++w) mx = fmaxf(mx, red[0][w][g]);
          M[g] = mx;
        }
        // this wave's positions 32 s + 4 wid + q, lane-parallel: e in f32 into
        // the denominator, the bf16 weight back over the score (0 past the context)
        for (int j = lane; j < 4 * nst; j += kWave) {
          const int pj = (j >> 2) * kSeqStep + 4 * wid + (j & 3);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float e = pj < n ? __builtin_amdgcn_exp2f((sc[g * npos + pj] - M[g]) * kLog2e) : 0.f;
            ls[g] += e;
            sc[g * npos + pj] = round_bf(e);
          }
        }
      }
    } else {
      const int pi = (c - nst) * kSeqStep + pw;
      if (c == nst + clast && pi == last) v = vnp;
      float vf[8];
      unpack8(v, vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float wgt = pi < n ? sc[g * npos + min(pi, n - 1)] : 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = fmaf(wgt, vf[i], o[g][i]);
      }
    }
  };
  for (int rd = 0; rd + 1 < nrounds; ++rd) {
#pragma unroll
    for (int r = 0; r < kSeqRing; ++r) {
      const int c = rd * kSeqRing + r;
      const uint4 v = ring[r];
      ring[r] = ld16_stream(chunk_ptr(min(c + kSeqRing, nch - 1)));
      step(c, v);
    }
  }
  // the last round issues no refills: none would be consumed, and the ring's
  // registers are reused after the loop (a load still in flight into them
  // would be waited for there)
#pragma unroll
  for (int r = 0; r < kSeqRing; ++r) step((nrounds - 1) * kSeqRing + r, ring[r]);

  // 4. the four position slots of a wave (row swaps), then the waves in order
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lw = wave_sum(ls[g]);   // the wave's positions sit one per lane
    if (lane == 0) red[1][wid][g] = lw;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = rows4_sum(o[g][i]);
  }
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < 8; ++i) obuf[wid][g][8 * dc + i] = o[g][i];
  }
  lds_barrier();
  for (int e = t; e < G * D; e += kSeqThreads) {
    const int g = e / D, d = e % D;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kSeqWaves; w += 2) {
      num += obuf[w][g][d] + obuf[w + 1][g][d];
      den += red[1][w][g] + red[1][w + 1][g];
    }
    ob[e] = static_cast<uint16_t>(f2bf(num / den));
  }
}

template <int G>
int launch_attn_seq_g(const AttnArgs& a, int batch, hipStream_t st) {
  using S = SeqShape<G>;
  if (static_cast<int64_t>(a.cap + S::step) * G > kSeqScores)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: cache of %d slots exceeds %d positions for group %d",
                a.cap, kSeqScores / G - S::step, G);
  attn_seq_kernel<G><<<dim3(a.hkv, batch), S::W * kWave, 0, st>>>(a, a.out);
  return launched("attn_seq");
}

template <int G, int NIT>
void launch_attn_mode(const AttnArgs& a, dim3 grid, hipStream_t st) {
  if (a.gq == nullptr) attn_decode_kernel<G, NIT, QM_PREPARED><<<grid, kThreads, 0, st>>>(a);
  else if (a.part == nullptr) attn_decode_kernel<G, NIT, QM_RAW><<<grid, kThreads, 0, st>>>(a);
  else attn_decode_kernel<G, NIT, QM_PART><<<grid, kThreads, 0, st>>>(a);
}

template <int G>
int launch_attn_g(const AttnArgs& a, int ss, int batch, hipStream_t st) {
  const dim3 grid(a.hkv, a.ns, batch);
  switch (ss) {
    case 32: launch_attn_mode<G, 2>(a, grid, st); break;
    case 64: launch_attn_mode<G, 4>(a, grid, st); break;
    case 128: launch_attn_mode<G, 8>(a, grid, st); break;
    case 256: launch_attn_mode<G, 16>(a, grid, st); break;
    default: return fail(TFA_ERR_SHAPE, "attn_decode: split %d not in {32, 64, 128, 256}", ss);
  }
  return launched("attn_decode");
}

// Merge: out[h*Dh + d] = bf16(sum_s op e^(mp-M) / sum_s lp e^(mp-M)). With wr,
// only the splits that hold slots <= wr[0] count. One block per head, one
// memory round trip: every load -- wr, one split's statistics per thread, and
// eight splits' partial outputs per thread -- is issued at the start (the
// partial outputs do not depend on the statistics, and splits past wr are read
// but never used: their rows are allocated, possibly stale). The block max and
// the denominator are tree reductions; eight groups of threads sum every eighth
// split and meet in LDS in group order.
constexpr int kCombThreads = 1024;
constexpr int kCombWaves = kCombThreads / kWave;
constexpr int kCombGroups = 8;
constexpr int kCombMaxSplits = kCombThreads;
constexpr int kCombMaxD = kCombThreads / kCombGroups;
constexpr int kCombUnroll = 8;

__global__ __launch_bounds__(kCombThreads) void attn_combine_kernel(
    const float* op, const float* mp, const float* lp, uint16_t* out, int ns, int hq, int Dh,
    const int* wr, int split) {
  const int bb = blockIdx.y;
  op += static_cast<size_t>(bb) * ns * hq * Dh;
  mp += static_cast<size_t>(bb) * ns * hq;
  lp += static_cast<size_t>(bb) * ns * hq;
  out += static_cast<size_t>(bb) * hq * Dh;
  __shared__ float s_e[kCombMaxSplits];
  __shared__ float s_red[kCombGroups][kCombMaxD];
  __shared__ float s_w[2][kCombWaves];
  const int h = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1), wid = t / kWave;
  const int gi = t / kCombMaxD;
  const int d = t % kCombMaxD;
  const int nsc = ns < kCombMaxSplits ? ns : kCombMaxSplits;
  // 1. every load of the first round, together
  const int w = wr ? wr[bb] : 0;
  const bool in = t < nsc;
  const float mj0 = in ? mp[t * hq + h] : -INFINITY;
  const float lj0 = in ? lp[t * hq + h] : 0.f;
  float v[kCombUnroll];
#pragma unroll
  for (int u = 0; u < kCombUnroll; ++u) {
    const int j = gi + u * kCombGroups;
    v[u] = (d < Dh && j < nsc) ? op[(static_cast<size_t>(j) * hq + h) * Dh + d] : 0.f;
  }
  int nact = nsc;
  if (wr) {
    nact = w < 0 ? 0 : w / split + 1;
    if (nact > nsc) nact = nsc;
  }
  // 2. statistics: block max, weights, denominator
  const bool act = t < nact;
  const float mj = act ? mj0 : -INFINITY;
  float mx = wave_max(mj);
  if (lane == 0) s_w[0][wid] = mx;
  lds_barrier();
  mx = s_w[0][0];
#pragma unroll
  for (int k = 1; k < kCombWaves; ++k) mx = fmaxf(mx, s_w[0][k]);
  const float e = act ? expf(mj - mx) : 0.f;
  s_e[t] = e;
  const float dw = wave_sum(act ? lj0 * e : 0.f);
  if (lane == 0) s_w[1][wid] = dw;
  lds_barrier();
  float den = 0.f;
#pragma unroll
  for (int k = 0; k < kCombWaves; ++k) den += s_w[1][k];
  // 3. partial outputs: group gi sums splits gi, gi + 8, ...
  if (d < Dh) {
    float num = 0.f;
#pragma unroll
    for (int u = 0; u < kCombUnroll; ++u) {
      const int j = gi + u * kCombGroups;
      if (j < nact) num = fmaf(v[u], s_e[j], num);
    }
    for (int j0 = gi + kCombGroups * kCombUnroll; j0 < nact; j0 += kCombGroups * kCombUnroll) {
      float x[kCombUnroll];
#pragma unroll
      for (int u = 0; u < kCombUnroll; ++u) {
        const int j = j0 + u * kCombGroups;
        x[u] = j < nact ? op[(static_cast<size_t>(j) * hq + h) * Dh + d] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kCombUnroll; ++u) {
        const int j = j0 + u * kCombGroups;
        if (j < nact) num = fmaf(x[u], s_e[j], num);
      }
    }
    s_red[gi][d] = num;
  }
  lds_barrier();
  if (t < Dh) {
    float num = 0.f;
#pragma unroll
    for (int g = 0; g < kCombGroups; ++g) num += s_red[g][t];
    out[h * Dh + t] = static_cast<uint16_t>(f2bf(num / den));
  }
}

// The merge for head_dim 128 and up to 128 splits, spread wider: block (head,
// 32-dim slice), 256 threads = 8 groups of 32 lanes, group g owning splits g,
// g + 8, ... and lane d one output dim. Every load a thread needs -- its splits'
// statistics and partial outputs, active or not (rows past wr are allocated,
// possibly stale, and never used) -- is issued at once, next to wr, so the whole
// merge is one memory round trip; the block max and the group sums meet in LDS
// in group order.
constexpr int kFastSlices = 4;                     // 32-dim slices of a 128-dim head
constexpr int kFastGroups = 8;
constexpr int kFastPer = 16;                       // splits per group
constexpr int kFastMaxSplits = kFastGroups * kFastPer;

__global__ __launch_bounds__(256) void attn_combine_d128_kernel(const float* op, const float* mp, const float* lp,
                                                                uint16_t* out, int ns, int hq, const int* wr,
                                                                int split) {
  const int h = blockIdx.x / kFastSlices, c = blockIdx.x % kFastSlices;
  const int bb = blockIdx.y;
  const int t = threadIdx.x, g = t / 32, d = 32 * c + (t & 31);
  op += static_cast<size_t>(bb) * ns * hq * D;
  mp += static_cast<size_t>(bb) * ns * hq;
  lp += static_cast<size_t>(bb) * ns * hq;
  __shared__ float s_m[kFastGroups];
  __shared__ float s_den[kFastGroups];
  __shared__ float s_num[kFastGroups][32];
  const int w = wr ? wr[bb] : 0;
  float m[kFastPer], l[kFastPer], o[kFastPer];
#pragma unroll
  for (int u = 0; u < kFastPer; ++u) {
    const int j = g + kFastGroups * u;
    const bool in = j < ns;
    m[u] = in ? mp[j * hq + h] : -INFINITY;
    l[u] = in ? lp[j * hq + h] : 0.f;
    o[u] = in ? op[(static_cast<size_t>(j) * hq + h) * D + d] : 0.f;
  }
  int nact = ns;
  if (wr) {
    nact = w < 0 ? 0 : w / split + 1;
    if (nact > ns) nact = ns;
  }
  float gm = -INFINITY;
#pragma unroll
  for (int u = 0; u < kFastPer; ++u)
    if (g + kFastGroups * u < nact) gm = fmaxf(gm, m[u]);
  if ((t & 31) == 0) s_m[g] = gm;
  lds_barrier();
  float M = s_m[0];
#pragma unroll
  for (int k = 1; k < kFastGroups; ++k) M = fmaxf(M, s_m[k]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int u = 0; u < kFastPer; ++u) {
    if (g + kFastGroups * u < nact) {
      const float e = expf(m[u] - M);
      num = fmaf(o[u], e, num);
      den = fmaf(l[u], e, den);
    }
  }
  s_num[g][t & 31] = num;
  if ((t & 31) == 0) s_den[g] = den;
  lds_barrier();
  if (g == 0) {
    float tn = 0.f, td = 0.f;
#pragma unroll
    for (int k = 0; k < kFastGroups; ++k) {
      tn += s_num[k][t & 31];
      td += s_den[k];
    }
    out[static_cast<size_t>(bb) * hq * D + h * D + d] = static_cast<uint16_t>(f2bf(tn / td));
  }
}

// combine_gemv: the split merge folded into the o_proj GEMV with its residual,
// for one sequence, hq <= 16 heads of 128 (K = hq * 128 <= 2048). A block of 16
// waves owns 8 RPW output rows. Every load is issued first: each wave's chunk
// of its rows' weights (wave (quarter q, pair group pg): 16-byte chunk `lane` of
// quarter q of RPW row pairs), then for wave h < hq its head's split statistics
// (lane s: split s) and its lane's two dims of the first kCgRound splits'
// partial rows. The merge is attn_combine_d128's arithmetic exactly -- the max
// over the active splits, e = expf(m - max), splits summed by fmaf in groups
// s % 8 (in s order within a group, the groups in order), one landing of
// num / den -- with each split's e and l broadcast by readlane; the merged
// vector goes to LDS (and, from block 0, to attn_out). The product is
// gemv_rows_kernel's for 2-row blocks exactly: per row pair one quarter per
// wave, one 16-byte chunk per lane, the wave's two-row transposed reduction,
// quarters summed (0 + 1) + (2 + 3), y = bf16(res + bf16(sum)). So the result
// is bit-identical to attn_combine followed by gemv_residual, one launch fewer.
// Every block re-reads the partials, 16 x (128 + 2) floats per split; more than
// kCgMaxSplits splits are refused (two launches). Measured in the Qwen3-1.7B
// bs=1 step (contexts 64..2112): 905 tok/s against 961 for the two launches with
// 8-row blocks, 897 / 846 with 16 / 32 rows -- the per-CU re-read costs more
// than the launch it saves, so the engine keeps two launches by default.
// Replaces examples/qwen3_1_7b-tilelang/fast/kernels.py:154-207 (gemv_attn_combine)
// with the residual add of ref_src/model.py:263.
constexpr int kCgWaves = 16;
constexpr int kCgThreads = kCgWaves * kWave;
constexpr int kCgMaxSplits = 64;   // one split's statistics per lane
constexpr int kCgRound = 32;       // splits whose partial rows are in flight at once

template <int RPW>
__global__ __launch_bounds__(kCgThreads) void combine_gemv_kernel(
    const float* op, const float* mp, const float* lp, int ns, int hq, const int* wr, int split,
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ res, uint16_t* __restrict__ y, int N,
    uint16_t* attn_out) {
  constexpr int RB = 8 * RPW;
  __shared__ float xs[16 * D];
  __shared__ float red[4][4][RPW][2];   // [pair group][quarter][pair][row of the pair]
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wid = t / kWave;
  const int K = hq * D;
  const int kq = K / 4;
  const int q = wid & 3, pg = wid >> 2;
  const int row0 = blockIdx.x * RB;
  const bool cvalid = 8 * lane < kq;

  // 1. the weights, the residual, the write slot, then the merge operands --
  //    every load unconditional at an in-bounds address (rows, chunks, heads
  //    and splits clamped; what they bring past the shape is never used), so
  //    they all go out before the first wait
  const int cl = min(lane, kq / 8 - 1);
  uint4 wv[RPW][2];
#pragma unroll
  for (int p = 0; p < RPW; ++p)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int row = min(row0 + (pg * RPW + p) * 2 + r, N - 1);
      wv[p][r] = ld16_stream(w + static_cast<size_t>(row) * K + q * kq + 8 * cl);
    }
  const float rv = bf2f(res[min(row0 + min(t, RB - 1), N - 1)]);
  const int wslot = wr ? wr[0] : 0;
  const int h = min(wid, hq - 1);
  const bool merger = wid < hq;
  const int sl = min(lane, ns - 1);
  const float m_l = mp[sl * hq + h];
  const float l_l = lp[sl * hq + h];
  float2 o[kCgRound];
#pragma unroll
  for (int s = 0; s < kCgRound; ++s)
    o[s] = *reinterpret_cast<const float2*>(op + (static_cast<size_t>(min(s, ns - 1)) * hq + h) * D + 2 * lane);

  // 2. the merge (wave h: dims 2 lane, 2 lane + 1 of head h)
  if (merger) {
    int nact = ns;
    if (wr) {
      nact = wslot < 0 ? 0 : wslot / split + 1;
      if (nact > ns) nact = ns;
    }
    const bool act = lane < nact;
    const float M = wave_max(act ? m_l : -INFINITY);
    const float e_l = act ? expf(m_l - M) : 0.f;
    float n0[8], n1[8], dg[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) n0[g] = n1[g] = dg[g] = 0.f;
    auto take = [&](int s, float2 v) __attribute__((always_inline)) {
      const float es = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e_l), s));
      const float ls = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_l), s));
      n0[s & 7] = fmaf(v.x, es, n0[s & 7]);
      n1[s & 7] = fmaf(v.y, es, n1[s & 7]);
      dg[s & 7] = fmaf(ls, es, dg[s & 7]);
    };
#pragma unroll
    for (int s = 0; s < kCgRound; ++s)
      if (s < nact) take(s, o[s]);
    if (nact > kCgRound) {   // wave-uniform: a second round of partial rows
#pragma unroll
      for (int s = 0; s < kCgRound; ++s)
        o[s] = *reinterpret_cast<const float2*>(
            op + (static_cast<size_t>(min(kCgRound + s, ns - 1)) * hq + h) * D + 2 * lane);
#pragma unroll
      for (int s = 0; s < kCgRound; ++s)
        if (kCgRound + s < nact) take(kCgRound + s, o[s]);
    }
    float tn0 = 0.f, tn1 = 0.f, td = 0.f;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      tn0 += n0[g];
      tn1 += n1[g];
      td += dg[g];
    }
    const uint32_t a0 = f2bf(tn0 / td), a1 = f2bf(tn1 / td);
    xs[h * D + 2 * lane] = bf2f(a0);
    xs[h * D + 2 * lane + 1] = bf2f(a1);
    if (attn_out && blockIdx.x == 0)
      *reinterpret_cast<uint32_t*>(attn_out + h * D + 2 * lane) = a0 | (a1 << 16);
  }
  lds_barrier();

  // 3. the product: wave (q, pg), row pairs pg * RPW + p
  float xf[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xf[i] = cvalid ? xs[q * kq + 8 * cl + i] : 0.f;
#pragma unroll
  for (int p = 0; p < RPW; ++p) {
    float acc[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float f[8];
      unpack8(cvalid ? wv[p][r] : make_uint4(0, 0, 0, 0), f);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) s = fmaf(xf[i], f[i], s);
      acc[r] = s;
    }
    const float tot = wave_sum_rows<2>(acc, lane);
    if ((lane & (kWave / 2 - 1)) == 0) red[pg][q][p][wave_rows_owner<2>(lane)] = tot;
  }
  lds_barrier();
  if (t < RB && row0 + t < N) {
    const int pr = t >> 1, rr = t & 1;
    const int g = pr / RPW, p = pr % RPW;
    const float v = (red[g][0][p][rr] + red[g][1][p][rr]) + (red[g][2][p][rr] + red[g][3][p][rr]);
    y[row0 + t] = static_cast<uint16_t>(f2bf(rv + round_bf(v)));
  }
}

template <int RPW>
int launch_combine_gemv(const float* op, const float* mp, const float* lp, int ns, int hq, const int* wr, int split,
                        const void* w_o, const void* residual, void* y, int n, void* attn_out, hipStream_t stream) {
  const unsigned blocks = static_cast<unsigned>((n + 8 * RPW - 1) / (8 * RPW));
  combine_gemv_kernel<RPW><<<blocks, kCgThreads, 0, stream>>>(
      op, mp, lp, ns, hq, wr, split, static_cast<const uint16_t*>(w_o), static_cast<const uint16_t*>(residual),
      static_cast<uint16_t*>(y), n, static_cast<uint16_t*>(attn_out));
  return launched("attn_combine_gemv_residual");
}

// qk_rope_cache: one wave per head of the [q | k | v] projection, summed from
// its split-K partials [ks, B, (hq + 2 hkv) * 128] and landed in bf16. Query
// heads get the per-head norm and RoPE at pos[b] and go to q_out; the key head
// gets the same with gamma_k and the value head nothing, and both are written
// to cache row wr[b]. The standalone form of the fused mode above, for callers
// that keep the prepared query (examples/qwen3_1_7b-tilelang/fast/kernels.py:328-411).
__global__ __launch_bounds__(kThreads) void qk_rope_cache_kernel(
    const float* __restrict__ part, int ks, const uint16_t* __restrict__ gq,
    const uint16_t* __restrict__ gk, float eps, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int mp_rows, const int* __restrict__ pos,
    const int* __restrict__ wr, uint16_t* kc, uint16_t* vc, int cap, uint16_t* q_out, int hq,
    int hkv, int* err) {
  const int lane = threadIdx.x & (kWave - 1);
  const int hh = blockIdx.x * kWaves + threadIdx.x / kWave;
  const int b = blockIdx.y;
  const int tot = hq + 2 * hkv;
  if (hh >= tot) return;  // whole waves only
  const int rows = tot * D;
  const size_t kstride = static_cast<size_t>(rows) * gridDim.y;
  float x0, x1;
  head_raw(nullptr, part + static_cast<size_t>(b) * rows + static_cast<size_t>(hh) * D, ks, kstride,
           lane, x0, x1);
  const size_t KN = static_cast<size_t>(hkv) * D;
  const int slot = wr[b];
  const bool slot_ok = slot >= 0 && slot < cap;
  if (hh >= hq + hkv) {
    if (!slot_ok) {
      if (lane == 0) set_err(err, 3);
      return;
    }
    uint16_t* dst = vc + (static_cast<size_t>(b) * cap + slot) * KN + (hh - hq - hkv) * D;
    dst[lane] = static_cast<uint16_t>(f2bf(x0));
    dst[lane + 64] = static_cast<uint16_t>(f2bf(x1));
    return;
  }
  int p = pos[b];
  if (p < 0 || p >= mp_rows) {
    if (lane == 0) set_err(err, 5);
    p = 0;
  }
  const size_t pr = static_cast<size_t>(p) * D;
  const float c0 = bf2f(cos_t[pr + lane]), s0 = bf2f(sin_t[pr + lane]);
  const float c1 = bf2f(cos_t[pr + lane + 64]), s1 = bf2f(sin_t[pr + lane + 64]);
  float o0, o1;
  norm_rope_head(x0, x1, hh < hq ? gq : gk, eps, c0, s0, c1, s1, lane, o0, o1);
  uint16_t* dst;
  if (hh < hq) {
    dst = q_out + (static_cast<size_t>(b) * hq + hh) * D;
  } else {
    if (!slot_ok) {
      if (lane == 0) set_err(err, 3);
      return;
    }
    dst = kc + (static_cast<size_t>(b) * cap + slot) * KN + (hh - hq) * D;
  }
  dst[lane] = static_cast<uint16_t>(f2bf(o0));
  dst[lane + 64] = static_cast<uint16_t>(f2bf(o1));
}

// prefill_qk_rope: the prompt rows of a q|k|v projection, the sum of ks f32
// split-K partials [ks, rows, ldq] with rows = batch * n (sequence b's row r
// at b * n + r, position pos0 + r).
// One wave per (row, head), the decode step's per-head arithmetic: land in
// bf16, query heads get the per-head norm and RoPE and go to q_out[row],
// the key head the same with gamma_k into cache row pos0 + r of sequence b,
// the value head straight into the value cache.
__global__ __launch_bounds__(kThreads) void prefill_qk_rope_kernel(
    const float* __restrict__ part, int ks, int64_t ldq, const uint16_t* __restrict__ gq,
    const uint16_t* __restrict__ gk, float eps, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int n, int pos0, uint16_t* kc, uint16_t* vc, int64_t cap,
    uint16_t* q_out, int hq, int hkv, int64_t rows) {
  const int lane = threadIdx.x & (kWave - 1);
  const int tot = hq + 2 * hkv;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
  if (w >= rows * tot) return;  // whole waves only
  const int64_t m = w / tot;
  const int hh = static_cast<int>(w % tot);
  const int64_t b = m / n;
  const int p = pos0 + static_cast<int>(m % n);
  float x0, x1;
  head_raw(nullptr, part + m * ldq + static_cast<int64_t>(hh) * D, ks, static_cast<size_t>(rows * ldq), lane, x0,
           x1);
  const int64_t KN = static_cast<int64_t>(hkv) * D;
  const int64_t crow = (b * cap + p) * KN;
  if (hh >= hq + hkv) {
    uint16_t* dst = vc + crow + (hh - hq - hkv) * D;
    dst[lane] = static_cast<uint16_t>(f2bf(x0));
    dst[lane + 64] = static_cast<uint16_t>(f2bf(x1));
    return;
  }
  const size_t pr = static_cast<size_t>(p) * D;
  const float c0 = bf2f(cos_t[pr + lane]), s0 = bf2f(sin_t[pr + lane]);
  const float c1 = bf2f(cos_t[pr + lane + 64]), s1 = bf2f(sin_t[pr + lane + 64]);
  float o0, o1;
  norm_rope_head(x0, x1, hh < hq ? gq : gk, eps, c0, s0, c1, s1, lane, o0, o1);
  uint16_t* dst = hh < hq ? q_out + (m * hq + hh) * D : kc + crow + (hh - hq) * D;
  dst[lane] = static_cast<uint16_t>(f2bf(o0));
  dst[lane + 64] = static_cast<uint16_t>(f2bf(o1));
}

}  // namespace

extern "C" {

int tfa_decode_attention(const void* q, const float* qkv_part, int64_t part_ks,
                         const void* gamma_q, const void* gamma_k, float eps_head,
                         const void* cos_t, const void* sin_t, int64_t rope_rows, void* k_cache,
                         void* v_cache, const int* pos, const int* wr, int64_t batch, int64_t hq,
                         int64_t hkv, int64_t head_dim, int64_t cap, int64_t split, float scale,
                         float* op, float* mp, float* lp, int neutral, int* err,
                         hipStream_t stream) {
  if (!k_cache || !v_cache || !wr || !op || !mp || !lp)
    return fail(TFA_ERR_NULL, "tfa_decode_attention: null pointer argument");
  if (!q && !qkv_part) return fail(TFA_ERR_NULL, "tfa_decode_attention: q or qkv_part required");
  if (head_dim != D) return fail(TFA_ERR_SHAPE, "tfa_decode_attention: head_dim %lld, only 128 supported", (long long)head_dim);
  if (hkv <= 0 || hq % hkv != 0) return fail(TFA_ERR_SHAPE, "tfa_decode_attention: hq %lld not a multiple of hkv %lld", (long long)hq, (long long)hkv);
  if (split <= 0 || cap <= 0 || cap % split != 0)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention: cap %lld not a positive multiple of split %lld", (long long)cap, (long long)split);
  if (batch < 1 || batch > 65535) return fail(TFA_ERR_SHAPE, "tfa_decode_attention: batch %lld out of range", (long long)batch);
  if ((q && !aligned16(q)) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(TFA_ERR_ALIGN, "tfa_decode_attention: q / caches not 16-byte aligned");
  if (gamma_q && (!gamma_k || !cos_t || !sin_t || !pos || rope_rows <= 0))
    return fail(TFA_ERR_NULL, "tfa_decode_attention: fused mode needs gamma_k, cos, sin, pos");
  if (qkv_part && (!gamma_q || part_ks < 1))
    return fail(TFA_ERR_ARG, "tfa_decode_attention: partials are a fused-mode source (gamma_q, ks >= 1)");
  if (qkv_part && part_ks > kMaxSplitsK)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention: part_ks %lld exceeds %d", (long long)part_ks, kMaxSplitsK);
  AttnArgs a{};
  a.q = qkv_part ? nullptr : static_cast<const uint16_t*>(q);
  a.part = qkv_part;
  a.part_ks = (int)part_ks;
  a.q_bstride = static_cast<size_t>(gamma_q ? hq + hkv : hq) * D;
  a.cache_bstride = static_cast<size_t>(cap) * hkv * D;
  a.gq = static_cast<const uint16_t*>(gamma_q);
  a.gk = static_cast<const uint16_t*>(gamma_k);
  a.eps_head = eps_head;
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.mp_rows = (int)rope_rows;
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.pos = pos;
  a.wr = wr;
  a.op = op;
  a.mp = mp;
  a.lp = lp;
  a.neutral = neutral;
  a.err = err;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.cap = (int)cap;
  if (cap / split > 65535)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention: %lld splits exceed 65535", (long long)(cap / split));
  a.ns = (int)(cap / split);
  a.scale = scale;
  const int B = (int)batch;
  switch (hq / hkv) {
    case 1: return launch_attn_g<1>(a, (int)split, B, stream);
    case 2: return launch_attn_g<2>(a, (int)split, B, stream);
    case 4: return launch_attn_g<4>(a, (int)split, B, stream);
    case 8: return launch_attn_g<8>(a, (int)split, B, stream);
    default: return fail(TFA_ERR_SHAPE, "tfa_decode_attention: group %lld not in {1,2,4,8}", (long long)(hq / hkv));
  }
}

int tfa_decode_attention_seq(const float* qkv_part, int64_t part_ks, const void* gamma_q,
                             const void* gamma_k, float eps_head, const void* cos_t, const void* sin_t,
                             int64_t rope_rows, void* k_cache, void* v_cache, const int* pos, const int* wr,
                             int64_t batch, int64_t hq, int64_t hkv, int64_t head_dim, int64_t cap, float scale,
                             void* out, int* err, hipStream_t stream) {
  if (!qkv_part || !gamma_q || !gamma_k || !cos_t || !sin_t || !k_cache || !v_cache || !pos || !wr || !out)
    return fail(TFA_ERR_NULL, "tfa_decode_attention_seq: null pointer argument");
  if (head_dim != D) return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: head_dim %lld, only 128 supported", (long long)head_dim);
  if (hkv <= 0 || hq % hkv != 0)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: hq %lld not a multiple of hkv %lld", (long long)hq, (long long)hkv);
  if (cap <= 0 || rope_rows <= 0) return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: empty cache or rope table");
  if (batch < 1 || batch > 65535) return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: batch %lld out of range", (long long)batch);
  if (part_ks < 1 || part_ks > kMaxSplitsK)
    return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: part_ks %lld not in [1, %d]", (long long)part_ks, kMaxSplitsK);
  if (!aligned16(k_cache) || !aligned16(v_cache))
    return fail(TFA_ERR_ALIGN, "tfa_decode_attention_seq: caches not 16-byte aligned");
  AttnArgs a{};
  a.part = qkv_part;
  a.part_ks = (int)part_ks;
  a.cache_bstride = static_cast<size_t>(cap) * hkv * D;
  a.gq = static_cast<const uint16_t*>(gamma_q);
  a.gk = static_cast<const uint16_t*>(gamma_k);
  a.eps_head = eps_head;
  a.cos_t = static_cast<const uint16_t*>(cos_t);
  a.sin_t = static_cast<const uint16_t*>(sin_t);
  a.mp_rows = (int)rope_rows;
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.pos = pos;
  a.wr = wr;
  a.out = static_cast<uint16_t*>(out);
  a.err = err;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.cap = (int)cap;
  a.scale = scale;
  const int B = (int)batch;
  switch (hq / hkv) {
    case 1: return launch_attn_seq_g<1>(a, B, stream);
    case 2: return launch_attn_seq_g<2>(a, B, stream);
    case 4: return launch_attn_seq_g<4>(a, B, stream);
    default:
      return fail(TFA_ERR_SHAPE, "tfa_decode_attention_seq: group %lld not in {1,2,4}", (long long)(hq / hkv));
  }
}

int tfa_attn_combine(const float* op, const float* mp, const float* lp, void* out, int64_t splits,
                     int64_t batch, int64_t hq, int64_t head_dim, const int* wr, int64_t split,
                     hipStream_t stream) {
  if (!op || !mp || !lp || !out) return fail(TFA_ERR_NULL, "tfa_attn_combine: null pointer argument");
  if (splits <= 0 || hq <= 0 || head_dim <= 0 || batch <= 0) return fail(TFA_ERR_SHAPE, "tfa_attn_combine: empty shape");
  if (wr && split <= 0) return fail(TFA_ERR_SHAPE, "tfa_attn_combine: split must be positive with wr");
  if (head_dim > kCombMaxD) return fail(TFA_ERR_SHAPE, "tfa_attn_combine: head_dim %lld exceeds %d", (long long)head_dim, kCombMaxD);
  if (splits > kCombMaxSplits) return fail(TFA_ERR_SHAPE, "tfa_attn_combine: %lld splits exceed %d", (long long)splits, kCombMaxSplits);
  if (head_dim == D && splits <= kFastMaxSplits) {
    attn_combine_d128_kernel<<<dim3((unsigned)(hq * kFastSlices), (unsigned)batch), 256, 0, stream>>>(
        op, mp, lp, static_cast<uint16_t*>(out), (int)splits, (int)hq, wr, (int)split);
    return launched("attn_combine");
  }
  const dim3 grid((unsigned)hq, (unsigned)batch);
  attn_combine_kernel<<<grid, kCombThreads, 0, stream>>>(op, mp, lp, static_cast<uint16_t*>(out),
                                                         (int)splits, (int)hq, (int)head_dim, wr,
                                                         (int)split);
  return launched("attn_combine");
}

int tfa_attn_combine_gemv_residual(const float* op, const float* mp, const float* lp, int64_t splits, int64_t hq,
                                   int64_t head_dim, const int* wr, int64_t split, const void* w_o,
                                   const void* residual, void* y, int64_t n, void* attn_out, hipStream_t stream) {
  if (!op || !mp || !lp || !w_o || !residual || !y)
    return fail(TFA_ERR_NULL, "tfa_attn_combine_gemv_residual: null pointer argument");
  if (head_dim != D) return fail(TFA_ERR_SHAPE, "tfa_attn_combine_gemv_residual: head_dim %lld, only 128 supported", (long long)head_dim);
  if (hq < 4 || hq > kCgWaves || hq % 4 != 0)
    return fail(TFA_ERR_SHAPE, "tfa_attn_combine_gemv_residual: hq %lld not a multiple of 4 in [4, %d]", (long long)hq, kCgWaves);
  if (splits < 1 || splits > kCgMaxSplits)
    return fail(TFA_ERR_SHAPE, "tfa_attn_combine_gemv_residual: %lld splits not in [1, %d]", (long long)splits, kCgMaxSplits);
  if (wr && split <= 0) return fail(TFA_ERR_SHAPE, "tfa_attn_combine_gemv_residual: split must be positive with wr");
  // up to 2560 rows the decode GEMV works in 2-row blocks, whose reduction this kernel repeats
  if (n < 1 || n > 2560) return fail(TFA_ERR_SHAPE, "tfa_attn_combine_gemv_residual: n %lld not in [1, 2560]", (long long)n);
  if (!aligned16(w_o) || !aligned16(op) || (attn_out && reinterpret_cast<uintptr_t>(attn_out) % 4 != 0))
    return fail(TFA_ERR_ALIGN, "tfa_attn_combine_gemv_residual: w_o / op not 16-byte aligned");
  return launch_combine_gemv<1>(op, mp, lp, (int)splits, (int)hq, wr, (int)split, w_o, residual, y, (int)n,
                                attn_out, stream);
}

int tfa_qk_rope_cache(const float* qkv_part, int64_t part_ks, const void* gamma_q,
                      const void* gamma_k, float eps_head, const void* cos_t, const void* sin_t,
                      int64_t rope_rows, const int* pos, const int* wr, void* k_cache,
                      void* v_cache, int64_t cap, void* q_out, int64_t batch, int64_t hq,
                      int64_t hkv, int64_t head_dim, int* err, hipStream_t stream) {
  if (!qkv_part || !gamma_q || !gamma_k || !cos_t || !sin_t || !pos || !wr || !k_cache ||
      !v_cache || !q_out)
    return fail(TFA_ERR_NULL, "tfa_qk_rope_cache: null pointer argument");
  if (head_dim != D) return fail(TFA_ERR_SHAPE, "tfa_qk_rope_cache: head_dim %lld, only 128 supported", (long long)head_dim);
  if (hq <= 0 || hkv <= 0 || cap <= 0 || rope_rows <= 0)
    return fail(TFA_ERR_SHAPE, "tfa_qk_rope_cache: empty heads, cache or rope table");
  if (part_ks < 1 || part_ks > kMaxSplitsK)
    return fail(TFA_ERR_SHAPE, "tfa_qk_rope_cache: part_ks %lld not in [1, %d]", (long long)part_ks, kMaxSplitsK);
  if (batch < 1 || batch > 65535) return fail(TFA_ERR_SHAPE, "tfa_qk_rope_cache: batch %lld out of range", (long long)batch);
  const dim3 grid((unsigned)((hq + 2 * hkv + kWaves - 1) / kWaves), (unsigned)batch);
  qk_rope_cache_kernel<<<grid, kThreads, 0, stream>>>(
      qkv_part, (int)part_ks, static_cast<const uint16_t*>(gamma_q),
      static_cast<const uint16_t*>(gamma_k), eps_head, static_cast<const uint16_t*>(cos_t),
      static_cast<const uint16_t*>(sin_t), (int)rope_rows, pos, wr, static_cast<uint16_t*>(k_cache),
      static_cast<uint16_t*>(v_cache), (int)cap, static_cast<uint16_t*>(q_out), (int)hq, (int)hkv, err);
  return launched("qk_rope_cache");
}

int tfa_prefill_qk_rope(const float* qkv, int64_t ldq, const void* gamma_q, const void* gamma_k, float eps_head,
                        const void* cos_t, const void* sin_t, int64_t rope_rows, int64_t batch, int64_t n,
                        int64_t pos0, void* k_cache, void* v_cache, int64_t cap, void* q_out, int64_t hq,
                        int64_t hkv, int64_t head_dim, hipStream_t stream) {
  return tfa_prefill_qk_rope_split(qkv, 1, ldq, gamma_q, gamma_k, eps_head, cos_t, sin_t, rope_rows, batch, n, pos0,
                                   k_cache, v_cache, cap, q_out, hq, hkv, head_dim, stream);
}

int tfa_prefill_qk_rope_split(const float* qkv, int64_t ks, int64_t ldq, const void* gamma_q, const void* gamma_k,
                              float eps_head, const void* cos_t, const void* sin_t, int64_t rope_rows,
                              int64_t batch, int64_t n, int64_t pos0, void* k_cache, void* v_cache, int64_t cap,
                              void* q_out, int64_t hq, int64_t hkv, int64_t head_dim, hipStream_t stream) {
  if (!qkv || !gamma_q || !gamma_k || !cos_t || !sin_t || !k_cache || !v_cache || !q_out)
    return fail(TFA_ERR_NULL, "tfa_prefill_qk_rope: null pointer argument");
  if (ks < 1 || ks > kMaxSplitsK)
    return fail(TFA_ERR_SHAPE, "tfa_prefill_qk_rope: ks %lld not in [1, %d]", (long long)ks, kMaxSplitsK);
  if (head_dim != D) return fail(TFA_ERR_SHAPE, "tfa_prefill_qk_rope: head_dim %lld, only 128 supported", (long long)head_dim);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return fail(TFA_ERR_SHAPE, "tfa_prefill_qk_rope: hq %lld not a multiple of hkv %lld", (long long)hq, (long long)hkv);
  if (batch < 1 || n < 1 || n > (1 << 24) || pos0 < 0 || pos0 > (1 << 24) || cap < 1)
    return fail(TFA_ERR_SHAPE, "tfa_prefill_qk_rope: batch, rows (at most 2^24), cache or pos0 out of range");
  if (ldq < (hq + 2 * hkv) * D)
    return fail(TFA_ERR_SHAPE, "tfa_prefill_qk_rope: ldq %lld below the %lld projection columns", (long long)ldq,
                (long long)((hq + 2 * hkv) * D));
  if (pos0 + n > cap)
    return fail(TFA_ERR_CAPACITY, "tfa_prefill_qk_rope: positions %lld..%lld exceed the cache capacity %lld",
                (long long)pos0, (long long)(pos0 + n - 1), (long long)cap);
  if (pos0 + n > rope_rows)
    return fail(TFA_ERR_CAPACITY, "tfa_prefill_qk_rope: positions up to %lld exceed the %lld rope rows",
                (long long)(pos0 + n - 1), (long long)rope_rows);
  const int64_t rows = batch * n;
  const int64_t waves = rows * (hq + 2 * hkv);
  if ((waves + kWaves - 1) / kWaves > INT32_MAX)
    return fail(TFA_ERR_SHAPE, "tfa_prefill_qk_rope: %lld rows too many", (long long)rows);
  prefill_qk_rope_kernel<<<(unsigned)((waves + kWaves - 1) / kWaves), kThreads, 0, stream>>>(
      qkv, (int)ks, ldq, static_cast<const uint16_t*>(gamma_q), static_cast<const uint16_t*>(gamma_k), eps_head,
      static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t), (int)n, (int)pos0,
      static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cap, static_cast<uint16_t*>(q_out),
      (int)hq, (int)hkv, rows);
  return launched("prefill_qk_rope");
}

}  // extern "C"
