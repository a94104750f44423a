// Dense bf16 GEMM for the prefill projections: C[M, N] = A[M, K] . B[N, K]^T
// (activations and weights both K-contiguous, f32 accumulate) on
// v_mfma_f32_32x32x16_bf16, with fused epilogues:
//
//   store         C = bf16(acc)
//   residual      C = bf16(R + bf16(acc))                      (o_proj + residual)
//   f32           C = acc, unrounded                           (prompt prefill; K may be
//                 split into ranges written as separate partial slices, which
//                 the consumers sum in split order)
//   qk_norm_rope  the qkv projection, laid out per token [q_0 | gate_0 | ... |
//                 q_{H-1} | gate_{H-1} | k_0 .. k_{G-1} | v_0 .. v_{G-1}], 256 per
//                 slice: q and k slices get the per-head RMSNorm with (1 + gamma)
//                 in f32 (from the bf16-landed projection) and rotate-half RoPE on
//                 their leading 64 dims (bf16 products and sum); gate and v slices
//                 are stored as the projection landed them.
//
// Block tiles (BM x BN x 64) and wave layouts are template parameters; a launch
// picks (see launch()):
//   256 x 256, 8 waves of 128 x 64, 2 LDS stages   (grids that fill their rounds)
//   128 x 128, 4 waves of  64 x 64, 2 LDS stages   (the rest; two blocks per CU)
//   128 x 256, 8 waves of  64 x 64, 3 LDS stages   (the qkv epilogue's fallback)
// Two waves share each SIMD in the 8-wave tiles, so one wave's LDS reads and
// barrier waits sit under the other's MFMAs.
//
// Main loop: A and B k-slices stream global -> LDS with global_load_lds_dwordx4
// (16 bytes per lane, no registers), in a ring of LDS stages, loads running
// stages - 1 tiles ahead. Rows of 8 16-byte chunks are stored at chunk
// ^ ((row >> 1) & 7), so the 32-row operand reads are conflict-free. Each wave
// streams its operands through a two-deep register ring: the reads for k-step
// ks + 1 are interleaved with the MFMAs of k-step ks.
//
// Epilogue (bf16 outputs): the tile lands in bf16 into LDS (rows padded by 32
// bytes), then each wave takes whole rows -- 4 elements per lane -- and applies
// the residual add or the head norm + RoPE there, writing 8 bytes per lane, so
// every global access is a full coalesced row. The f32 store goes straight from
// the accumulators.
//
// Blocks are ordered for the L2s: the dispatcher deals blocks to the 8 XCDs in
// turn, so block b is renumbered to give each XCD a contiguous run of tiles,
// and tiles are numbered in groups of 8 block-rows so that the blocks one XCD
// runs together share A and B k-slices (+17 % on the 8192-token qkv over
// groups of 4).
//
// Reference (jingchangshi/TileFoundry): examples/qwen3_8_27b_prefill-tilelang/kernels/gemm.py:104-356
// (gemm_kernel, "qk_norm_rope" epilogue :226-300, "residual" :193-198), model.py:271-303,326-333.
#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kBK = 64;
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

TFA_DEV bf16x8 as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_F32 = 2, EPI_QKNR = 3 };

// sched_group_barrier instruction classes
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

struct GemmArgs {
  const uint16_t* a;      // [M, lda]
  const uint16_t* b;      // [N, ldb]
  uint16_t* c;            // [M, ldc]
  float* cf;              // [M, ldc] (f32 store)
  int M, N, K, lda, ldb, ldc;
  const uint16_t* res;    // residual [M, ldr]
  int ldr;
  const uint16_t* gq;     // q / k head norm weights [256] (the norm scales by 1 + gamma)
  const uint16_t* gk;
  const uint16_t* cos_t;  // [M, 64] rows = positions
  const uint16_t* sin_t;
  int heads, kv_heads;
  float eps;
  int ksplit;             // f32 store: K split into ksplit ranges, range z -> cf + z * M * ldc
};

TFA_DEV int swz(int row) { return (row >> 1) & 7; }

// Block b's tile (tm, tn) of an nm x nn grid: XCD-contiguous renumbering
// (XCD = true), then groups of GM tile rows walked column by column.
template <int GM, bool XCD>
TFA_DEV void tile_of(int b, int nm, int nn, int& tm, int& tn) {
  const int nb = nm * nn;
  int t = b;
  if (XCD) {
    const int per = nb / kXcds, rem = nb % kXcds;
    const int x = b % kXcds, i = b / kXcds;
    t = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i;
  }
  const int group = t / (GM * nn);
  const int first = group * GM;
  const int gsz = min(nm - first, GM);
  const int in = t % (GM * nn);
  tm = first + in % gsz;
  tn = in / gsz;
}

// BM x BN block tile of WM x WN waves, S LDS stages; GM tile rows per group,
// XCD-contiguous block order, and the interleaved operand-read schedule.
template <int BM_, int BN_, int WM_, int WN_, int S_, int GM_ = kGroupM, bool XCD_ = true, bool SCHED_ = true,
          bool PRIO_ = false>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, S = S_, GM = GM_;
  static constexpr bool XCD = XCD_, SCHED = SCHED_, PRIO = PRIO_;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kWTM = BM / WM, kWTN = BN / WN;    // wave tile
  static constexpr int kTI = kWTM / 32, kTJ = kWTN / 32;  // MFMA tiles per wave
  static constexpr int kRows = BM + BN;                   // LDS rows per stage: A rows, then B rows
  static constexpr int kStage = kRows * kBK;              // elements per stage
  static constexpr int kDma = kRows * 8 / kWave / kWaves; // DMA instructions per wave per stage
  static constexpr int kEpPitch = BN + 16;                // epilogue LDS row pitch (elements)
  static constexpr int kSmem = (S * kStage > BM * kEpPitch ? S * kStage : BM * kEpPitch);
  static_assert(kDma * kWaves * 8 == kRows, "whole DMA instructions per wave");
  static_assert(kWTM % 32 == 0 && kWTN % 32 == 0, "wave tiles of whole 32 x 32 MFMA tiles");
  static_assert(kSmem * 2 <= 160 * 1024, "LDS budget");
  static_assert(BN == 128 || BN == 256, "the epilogue's row pass covers 128 or 256 columns");
};

using C256 = Cfg<256, 256, 2, 4, 2, 8>;  // 8 waves of 128 x 64; groups of 8 tile rows
using C128x256 = Cfg<128, 256, 2, 4, 3>; // 8 waves of 64 x 64
using C128 = Cfg<128, 128, 2, 2, 2>;     // 4 waves of 64 x 64, two blocks per CU

constexpr int kWaitVm0 = waitcnt_vm(0);

template <class C, int EPI>
__global__ __launch_bounds__(C::kThreads) void gemm_kernel(const GemmArgs a) {
  constexpr int BM = C::BM, BN = C::BN, S = C::S, TI = C::kTI, TJ = C::kTJ;
  __shared__ __attribute__((aligned(1024))) uint16_t smem[C::kSmem];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int n32 = lane & 31;
  const int kg = lane >> 5;
  const int wm = (wid / C::WN) * C::kWTM, wn = (wid % C::WN) * C::kWTN;
  const int nm = (a.M + BM - 1) / BM, nn = a.N / BN;
  int tm, tn;
  tile_of<C::GM, C::XCD>(blockIdx.x, nm, nn, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // Stage loads: DMA instruction j fills stage rows 8j .. 8j+7 (A rows 0..BM-1,
  // then B rows); lane l lands at row 8j + l/8, chunk slot l % 8, and so loads
  // logical chunk (l % 8) ^ swz(row). Wave w issues j = kDma w .. kDma w + kDma - 1.
  // Rows past M read row M - 1 (never stored).
  const uint16_t* src[C::kDma];
#pragma unroll
  for (int i = 0; i < C::kDma; ++i) {
    const int row = 8 * (C::kDma * wid + i) + (lane >> 3);
    const int q = (lane & 7) ^ swz(row);
    src[i] = row < BM ? a.a + static_cast<size_t>(min(m0 + row, a.M - 1)) * a.lda + 8 * q
                      : a.b + static_cast<size_t>(n0 + row - BM) * a.ldb + 8 * q;
  }
  auto load_stage = [&](int kt, int st) __attribute__((always_inline)) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < C::kDma; ++i)
      lds_dma16(src[i] + k0, lds_offset(&smem[st * C::kStage + 8 * (C::kDma * wid + i) * kBK]));
  };

  f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // f32 store with a split K: block row z of the grid takes k-tiles
  // [z nk / ksplit, (z + 1) nk / ksplit) and writes its own partial slice
  int nk = a.K / kBK;
  int kt0 = 0;
  if (EPI == EPI_F32 && a.ksplit > 1) {
    nk /= a.ksplit;
    kt0 = blockIdx.y * nk;
  }
  const int sx = swz(n32);   // every operand row this lane reads is wm (or BM + wn) + 32 i + n32
#pragma unroll
  for (int s0 = 0; s0 < S - 1; ++s0)
    if (s0 < nk) load_stage(kt0 + s0, s0);
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt % S;
    // this wave's loads of tile kt landed (vector-memory loads complete in
    // order); with three stages those of tile kt + 1 may still fly
    if (S > 2 && kt + S - 2 < nk) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(C::kDma * (S - 2)));
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
    }
    block_barrier();   // every wave's tile kt landed; every wave is done with tile kt - 1's stage
    if (kt + S - 1 < nk) load_stage(kt0 + kt + S - 1, (kt + S - 1) % S);

    const uint16_t* abase = &smem[st * C::kStage + (wm + n32) * kBK];
    const uint16_t* bbase = &smem[st * C::kStage + (BM + wn + n32) * kBK];
    uint4 aop[2][TI], bop[2][TJ];
    auto rd = [&](int ks, int slot) __attribute__((always_inline)) {
      const int off = 8 * ((2 * ks + kg) ^ sx);
#pragma unroll
      for (int i = 0; i < TI; ++i) aop[slot][i] = *reinterpret_cast<const uint4*>(abase + 32 * i * kBK + off);
#pragma unroll
      for (int j = 0; j < TJ; ++j) bop[slot][j] = *reinterpret_cast<const uint4*>(bbase + 32 * j * kBK + off);
    };
    rd(0, 0);
    if (C::PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      if (ks + 1 < kBK / 16) rd(ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(aop[ks & 1][i]), as_bf8(bop[ks & 1][j]),
                                                              acc[i][j], 0, 0, 0);
    }
    if (C::PRIO) __builtin_amdgcn_s_setprio(0);
    // order: k-step 0's operand reads, then each k-step's MFMAs with the next
    // k-step's reads spread between them
    constexpr int kReads = TI + TJ, kMfma = TI * TJ;
    constexpr int kPer = kMfma / kReads > 0 ? kMfma / kReads : 1;
    if (C::SCHED) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kReads, 0);
#pragma unroll
    for (int ks = 0; ks < kBK / 16 && C::SCHED; ++ks) {
      if (ks + 1 < kBK / 16) {
#pragma unroll
        for (int r = 0; r < kReads; ++r) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, kPer, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
        if (kMfma > kPer * kReads) __builtin_amdgcn_sched_group_barrier(kSchedMfma, kMfma - kPer * kReads, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, kMfma, 0);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm0);   // no load may still be writing this block's LDS

  // acc[i][j][4t + r]: tile row wm + 32 i + 8 t + 4 kg + r, column wn + 32 j + n32
  if (EPI == EPI_F32) {
    float* cf = a.cf + static_cast<size_t>(blockIdx.y) * a.M * a.ldc;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm + 32 * i + 8 * t + 4 * kg + r;
          if (row >= a.M) continue;
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            cf[static_cast<size_t>(row) * a.ldc + n0 + wn + 32 * j + n32] = acc[i][j][4 * t + r];
        }
    return;
  }

  // bf16 tile into LDS (rows padded by 16 elements), then whole rows out
  block_barrier();   // every wave's last operand reads are consumed: the stages are free
  uint16_t* ep = smem;
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ep[(wm + 32 * i + 8 * t + 4 * kg + r) * C::kEpPitch + wn + 32 * j + n32] =
              static_cast<uint16_t>(f2bf(acc[i][j][4 * t + r]));
  lds_barrier();

  constexpr int kLPR = BN / 4;          // lanes per row, 4 elements each
  constexpr int kRPP = kWave / kLPR;    // rows per wave pass
  const int sub = lane / kLPR, cl = (lane % kLPR) * 4;
  // q / k slice of the qkv projection (256 columns: the whole tile)
  bool norm = false;
  const uint16_t* gamma = nullptr;
  if (EPI == EPI_QKNR) {
    const int sl = n0 / 256;
    if (sl < 2 * a.heads) {
      norm = (sl & 1) == 0;
      gamma = a.gq;
    } else if (sl < 2 * a.heads + a.kv_heads) {
      norm = true;
      gamma = a.gk;
    }
  }
  float g4[4] = {0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_QKNR && norm) {
    const uint2 gv = *reinterpret_cast<const uint2*>(gamma + cl);
    g4[0] = lo_bf(gv.x); g4[1] = hi_bf(gv.x); g4[2] = lo_bf(gv.y); g4[3] = hi_bf(gv.y);
  }
  // Every global input of the row passes -- the residual rows, or the rope rows
  // of a q / k slice -- is issued before the first pass, into the registers the
  // accumulators held: one memory round trip for the epilogue instead of one per
  // pass (a one-round grid otherwise ends on 16-32 serial trips per block).
  constexpr int kPasses = BM / (C::kWaves * kRPP);
  static_assert(kPasses * C::kWaves * kRPP == BM, "whole row passes per wave");
  auto pass_row = [&](int p) __attribute__((always_inline)) { return wid * kRPP + p * C::kWaves * kRPP + sub; };
  uint2 pre_a[EPI == EPI_RESID || EPI == EPI_QKNR ? kPasses : 1];
  uint2 pre_b[EPI == EPI_QKNR ? kPasses : 1];
  if (EPI == EPI_RESID) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int grow = min(m0 + pass_row(p), a.M - 1);
      pre_a[p] = *reinterpret_cast<const uint2*>(a.res + static_cast<size_t>(grow) * a.ldr + n0 + cl);
    }
  }
  if (EPI == EPI_QKNR && norm && lane < 16) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int grow = min(m0 + pass_row(p), a.M - 1);
      pre_a[p] = *reinterpret_cast<const uint2*>(a.cos_t + static_cast<size_t>(grow) * 64 + 4 * lane);
      pre_b[p] = *reinterpret_cast<const uint2*>(a.sin_t + static_cast<size_t>(grow) * 64 + 4 * lane);
    }
  }
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int row = pass_row(p);
    const int grow = m0 + row;
    if (EPI == EPI_QKNR) {
      if (m0 + row - sub >= a.M) break;    // wave-uniform: one row per pass at BN = 256
    } else if (grow >= a.M) {
      continue;
    }
    uint2 v = *reinterpret_cast<const uint2*>(ep + row * C::kEpPitch + cl);
    uint16_t* dst = a.c + static_cast<size_t>(grow) * a.ldc + n0 + cl;
    if (EPI == EPI_RESID) {
      const uint2 rv = pre_a[p];
      v.x = pack_bf(round_bf(lo_bf(rv.x) + lo_bf(v.x)), round_bf(hi_bf(rv.x) + hi_bf(v.x)));
      v.y = pack_bf(round_bf(lo_bf(rv.y) + lo_bf(v.y)), round_bf(hi_bf(rv.y) + hi_bf(v.y)));
    }
    if (EPI == EPI_QKNR && norm) {
      // x -> bf16(x * rsqrt(mean x^2 + eps) * (1 + gamma)) in f32; then rotate-half
      // on dims 0..63, partners 32 apart (lane l and l ^ 8), products and sum in bf16
      const float x[4] = {lo_bf(v.x), hi_bf(v.x), lo_bf(v.y), hi_bf(v.y)};
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
      const float inv = rsqrt_rn(wave_sum(ss) / 256.0f + a.eps);
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = round_bf(x[i] * inv * (1.0f + g4[i]));
      float partner[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) partner[i] = xor_lane<8>(y[i], lane);
      if (lane < 16) {
        const uint2 cv = pre_a[p];
        const uint2 sv = pre_b[p];
        const float c[4] = {lo_bf(cv.x), hi_bf(cv.x), lo_bf(cv.y), hi_bf(cv.y)};
        const float s4[4] = {lo_bf(sv.x), hi_bf(sv.x), lo_bf(sv.y), hi_bf(sv.y)};
        const float sign = lane < 8 ? -1.0f : 1.0f;   // rotate_half: first half pairs with -x[d + 32]
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = round_bf(round_bf(y[i] * c[i]) + round_bf(sign * partner[i] * s4[i]));
      }
      v = make_uint2(pack_bf(y[0], y[1]), pack_bf(y[2], y[3]));
    }
    *reinterpret_cast<uint2*>(dst) = v;
  }
}

template <class C, int EPI>
int launch_cfg(const GemmArgs& g, hipStream_t st, const char* name) {
  const int nm = (g.M + C::BM - 1) / C::BM, nn = g.N / C::BN;
  const unsigned splits = EPI == EPI_F32 && g.ksplit > 1 ? (unsigned)g.ksplit : 1u;
  gemm_kernel<C, EPI><<<dim3((unsigned)(nm * nn), splits), C::kThreads, 0, st>>>(g);
  return launched(name);
}

// Tile choice. A 256 x 256 tile moves the fewest LDS bytes per FLOP and, at a
// full round of blocks, runs fastest (measured 1.10-1.15 PFLOP/s on the prefill
// shapes); but blocks run in rounds of one per CU, so a grid whose last round is
// mostly empty (320 blocks on 256 CUs: 62 % of two rounds) loses more than the
// smaller tile costs. Below 80 % round efficiency the 128 x 128 tile (two
// blocks per CU) takes over; the qkv + head-norm epilogue needs whole 256-column
// slices, so it falls back to 128 x 256 instead.
bool full_rounds_256(int64_t m, int64_t n, int cus) {
  const int64_t b256 = (m + 255) / 256 * (n / 256);
  const int64_t rounds = (b256 + cus - 1) / cus;
  return n % 256 == 0 && b256 * 5 >= rounds * cus * 4;
}

// K splits for the f32 store: a small grid (few token rows) of 128 x 128 tiles
// is split along K -- doubling while the blocks still fit twice per CU, each
// range keeps at least 4 k-tiles, and the count divides the k-tiles -- up to 8.
// The split count sets the order the consumers sum the partials in, and so the
// rounding of everything after the prompt prefill; it is therefore derived from
// the shape and MI355X's fixed 256 CUs, never from the device's reported count,
// so that a given prompt prefills to the same bits on any gfx950 part.
constexpr int kSplitPlanCus = 256;

int64_t splits_f32(int64_t m, int64_t n, int64_t k) {
  const int cus = kSplitPlanCus;
  if (full_rounds_256(m, n, cus) || n % 128 || k % kBK) return 1;
  const int64_t blocks = (m + 127) / 128 * (n / 128), nk = k / kBK;
  int64_t ks = 1;
  while (ks < kMaxSplitsK && blocks * ks * 2 <= 2 * cus && nk % (ks * 2) == 0 && nk / (ks * 2) >= 4) ks *= 2;
  return ks;
}

template <int EPI>
int launch(const GemmArgs& g, hipStream_t st, const char* name) {
  const int cus = device_cus();
  if (full_rounds_256(g.M, g.N, cus) && !(EPI == EPI_F32 && g.ksplit > 1)) return launch_cfg<C256, EPI>(g, st, name);
  if (EPI == EPI_QKNR) {
    if (g.N % 256) return fail(TFA_ERR_SHAPE, "%s: the qkv width must be a multiple of 256", name);
    return launch_cfg<C128x256, EPI>(g, st, name);
  }
  return launch_cfg<C128, EPI == EPI_QKNR ? EPI_STORE : EPI>(g, st, name);
}

int check_gemm(const void* a, const void* b, const void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
               int64_t ldc, const char* fn) {
  if (!a || !b || !c) return fail(TFA_ERR_NULL, "%s: null pointer argument", fn);
  if (m < 1 || n < 128 || n % 128 || k < kBK || k % kBK || m > (1 << 24) || n > (1 << 24) || k > (1 << 24))
    return fail(TFA_ERR_SHAPE, "%s: m %lld must be positive, n %lld a multiple of 128, k %lld of 64", fn,
                (long long)m, (long long)n, (long long)k);
  if (lda < k || ldb < k || ldc < n || lda % 8 || ldb % 8 || ldc % 4)
    return fail(TFA_ERR_SHAPE, "%s: leading dimensions too small, or lda / ldb not multiples of 8, ldc of 4", fn);
  if (!aligned16(a) || !aligned16(b)) return fail(TFA_ERR_ALIGN, "%s: a / b not 16-byte aligned", fn);
  if ((reinterpret_cast<uintptr_t>(c) & 7u) != 0) return fail(TFA_ERR_ALIGN, "%s: c not 8-byte aligned", fn);
  return TFA_OK;
}

GemmArgs make(const void* a, const void* b, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc) {
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a);
  g.b = static_cast<const uint16_t*>(b);
  g.M = (int)m; g.N = (int)n; g.K = (int)k;
  g.lda = (int)lda; g.ldb = (int)ldb; g.ldc = (int)ldc;
  return g;
}

}  // namespace

extern "C" {

int tfa_gemm_nt(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                int64_t ldc, const void* residual, int64_t ldr, hipStream_t stream) {
  const int st = check_gemm(a, b, c, m, n, k, lda, ldb, ldc, "tfa_gemm_nt");
  if (st != TFA_OK) return st;
  GemmArgs g = make(a, b, m, n, k, lda, ldb, ldc);
  g.c = static_cast<uint16_t*>(c);
  if (residual) {
    TFA_REQUIRE(ldr >= n && ldr % 4 == 0, TFA_ERR_SHAPE, "tfa_gemm_nt: ldr %lld < n %lld or not a multiple of 4",
                (long long)ldr, (long long)n);
    TFA_REQUIRE((reinterpret_cast<uintptr_t>(residual) & 7u) == 0, TFA_ERR_ALIGN,
                "tfa_gemm_nt: residual not 8-byte aligned");
    g.res = static_cast<const uint16_t*>(residual);
    g.ldr = (int)ldr;
    return launch<EPI_RESID>(g, stream, "gemm_nt_residual");
  }
  return launch<EPI_STORE>(g, stream, "gemm_nt");
}

int tfa_gemm_nt_f32(const void* a, const void* b, float* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                    int64_t ldb, int64_t ldc, hipStream_t stream) {
  return tfa_gemm_nt_f32_split(a, b, c, m, n, k, lda, ldb, ldc, 1, stream);
}

int64_t tfa_gemm_f32_splits(int64_t m, int64_t n, int64_t k) { return splits_f32(m, n, k); }

int tfa_gemm_nt_f32_split(const void* a, const void* b, float* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                          int64_t ldb, int64_t ldc, int64_t ks, hipStream_t stream) {
  const int st = check_gemm(a, b, c, m, n, k, lda, ldb, ldc, "tfa_gemm_nt_f32");
  if (st != TFA_OK) return st;
  TFA_REQUIRE(ks >= 1 && ks <= kMaxSplitsK && (k / kBK) % ks == 0, TFA_ERR_SHAPE,
              "tfa_gemm_nt_f32: %lld splits must be in [1, %d] and divide the %lld k-tiles of 64", (long long)ks,
              kMaxSplitsK, (long long)(k / kBK));
  GemmArgs g = make(a, b, m, n, k, lda, ldb, ldc);
  g.cf = c;
  g.ksplit = (int)ks;
  return launch<EPI_F32>(g, stream, "gemm_nt_f32");
}

int tfa_qkv_norm_rope(const void* hn, const void* w_qkv, void* out, int64_t n, int64_t hidden, int64_t heads,
                      int64_t kv_heads, int64_t head_dim, const void* gamma_q, const void* gamma_k, float eps,
                      const void* cos_t, const void* sin_t, int64_t rot, hipStream_t stream) {
  TFA_REQUIRE(head_dim == 256, TFA_ERR_SHAPE, "tfa_qkv_norm_rope: head_dim %lld, only 256 supported", (long long)head_dim);
  TFA_REQUIRE(rot == 64, TFA_ERR_SHAPE, "tfa_qkv_norm_rope: rot %lld, only 64 supported", (long long)rot);
  TFA_REQUIRE(heads >= 1 && kv_heads >= 1 && heads <= 4096 && kv_heads <= 4096, TFA_ERR_SHAPE,
              "tfa_qkv_norm_rope: head counts out of range");
  TFA_NONNULL(gamma_q);
  TFA_NONNULL(gamma_k);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  const int64_t width = (2 * heads + 2 * kv_heads) * head_dim;
  const int st = check_gemm(hn, w_qkv, out, n, width, hidden, hidden, hidden, width, "tfa_qkv_norm_rope");
  if (st != TFA_OK) return st;
  GemmArgs g = make(hn, w_qkv, n, width, hidden, hidden, hidden, width);
  g.c = static_cast<uint16_t*>(out);
  g.gq = static_cast<const uint16_t*>(gamma_q);
  g.gk = static_cast<const uint16_t*>(gamma_k);
  g.cos_t = static_cast<const uint16_t*>(cos_t);
  g.sin_t = static_cast<const uint16_t*>(sin_t);
  g.heads = (int)heads;
  g.kv_heads = (int)kv_heads;
  g.eps = eps;
  return launch<EPI_QKNR>(g, stream, "qkv_norm_rope");
}

}  // extern "C"
