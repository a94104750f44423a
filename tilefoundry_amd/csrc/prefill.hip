// Causal GQA prefill attention on bf16 MFMA, in two forms:
//
//   tfa_prefill_attention  head_dim 256 with the output gate (Qwen3.5-family
//                          full-attention layer, Qwen3.8-27B shapes: 24 query
//                          heads over 4 key/value heads), one sequence, n a
//                          multiple of 128;
//   tfa_causal_attention   head_dim 128 or 256, no gate, a batch of sequences
//                          of any length n (the prompt prefill of a decode
//                          model: Qwen3-1.7B shapes, 16 query heads over 8,
//                          K and V read straight from the decode cache).
//
// One block per (query head, 128 or 256 query rows, sequence): each wave (two
// per SIMD) owns 32 query rows over the whole head dimension and walks the
// 32-key tiles up to its diagonal -- or, in 128-row blocks at head_dim 256 on
// small grids, every other one of them, the two wave groups of the block
// merging their softmax states at the end. Per tile:
//
//   S^T = K . Q^T     v_mfma_f32_32x32x16_bf16, M = 32 keys, N = 32 queries,
//                     D/16 k-steps; Q^T is resident as the B operand, the
//                     K operands stream from LDS through a ring of registers
//                     (each read issued four k-steps ahead of its MFMA).
//   online softmax    per query (the MFMA output column): the lane holds 16
//                     of the tile's keys, its partner lane (l ^ 32) the other
//                     16 -- one exchange for the row max; exp2 with the scale
//                     folded in; the running max is only raised (and O
//                     rescaled) when a row's max passes it by more than 2^8.
//   O^T += V^T . P^T  M = 32 value dims (D/32 tiles), K = 16 keys per
//                     step; P^T is the bf16 score accumulator (its key slots
//                     relabelled), V^T comes from ds_read_b64_tr_b16 transpose
//                     reads of the row-major V tile, also streamed ahead.
//
// K and V tiles stream global -> LDS with global_load_lds_dwordx4 (no register
// staging) through two or three stages: the next tile's loads go out right
// after the tile barrier and land while this tile is computed. Each stage is
// its own LDS object and the block barrier is a bare s_barrier after an
// explicit wait for this wave's loads. At D = 256: 70 KB of LDS and at most
// 256 registers per wave for 128-row blocks, so two blocks share a CU (two
// waves per SIMD): one block's softmax and barrier waits run under the
// other's MFMAs. The output accumulators (D dims x 32 queries, f32) and Q stay
// in registers. Rows past n (a ragged last tile) read row n - 1 and are not
// stored.
// Epilogue in the reference's order: out = bf16(bf16(o / l) * bf16(sigmoid(gate)))
// with the gate, out = bf16(o / l) without.
//
// Reference (jingchangshi/TileFoundry): examples/qwen3_8_27b_prefill-tilelang/model.py:305-324
// (Attention.attention), kernels/attention.py:1-19,313-438 (attention_ws / attention_tir);
// the ungated form computes the attention of examples/qwen3_1_7b-tilelang/ref_src/model.py:171-215
// for every prompt row at once (the reference walks the prompt one decode step at a time,
// fast/engine.py:261-263).
#include <float.h>

#include <type_traits>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kBN = 32;             // keys per tile

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

TFA_DEV bf16x8 as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

struct FlashArgs {
  const uint16_t* q;     // element (b, n, h, d) at q + b*q_bs + n*q_rs + h*q_hs + d
  const uint16_t* k;     // (b, n, g, d) at k + b*k_bs + n*k_rs + g*k_hs + d
  const uint16_t* v;
  const uint16_t* gate;  // like q (gated form only)
  uint16_t* out;         // (b, n, h*D + d) at out + b*o_bs + n*o_rs + h*D + d
  int64_t q_bs, k_bs, v_bs, g_bs, o_bs;
  int q_rs, q_hs, k_rs, k_hs, v_rs, v_hs, g_rs, g_hs, o_rs;
  int N, HQ, HKV;        // N query rows (= keys) per sequence; any N >= 1
  int xcd_heads;         // heads per XCD in the work order (0: plain order)
  float scale_log2;      // head_dim^-1/2 * log2(e)
};

// LDS tiles hold one key per row, unpadded, so one DMA instruction fills 1 KB
// (2 rows at head_dim 256, 4 at 128). Each row's 16-byte chunks are XOR-
// swizzled instead: K row r by (r & 15), so the K operand read (16 rows, one
// chunk each per 16 lanes) hits 16 distinct bank quads; V row r by 4 (r & 3),
// so the transpose reads (4 rows x 64 bytes per 32 lanes) cover the 64 banks
// once. Every operand address is one per-lane base plus an immediate offset.
// sched_group_barrier instruction classes
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

TFA_DEV uint2 ld_tr(const uint16_t* lds_elem) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_elem));
  return __builtin_bit_cast(uint2, v);
}

constexpr int kWaitVm0 = waitcnt_vm(0);

// This wave's LDS writes are visible to its other lanes (LDS operations of one
// wave complete in order; the fences keep the compiler from moving them).
TFA_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Epilogue staging: each output wave's 32 rows x 64 dims of bf16(o / l) at a
// time, rows padded by 8 elements (the 32 rows' 8-byte writes spread over the
// banks), so that the gate is read and the output written as 16-byte pieces of
// whole rows (128 contiguous bytes per row, eight rows per instruction).
constexpr int kEpiDims = 64;
constexpr int kEpiPitch = kEpiDims + 8;

template <int N>
using IC = std::integral_constant<int, N>;

// W waves of 32 query rows per block, times KG key groups. W = 8 (256 rows, 3
// stages, one block per CU) halves the K/V bytes moved into LDS per FLOP
// against W = 4 (128 rows, 2 stages, two blocks per CU); both keep two waves
// per SIMD. KG = 2 (with W = 4) splits the keys of one 128-row tile between two
// wave groups over the same rows: group g takes key tiles g, g + 2, ..., each
// step brings one tile per group, and the groups' (max, sum, output) merge
// through LDS at the end. That halves the longest walk of a block, keeps two
// waves per SIMD with one block per CU, and makes the causal work finer
// grained, so the grid balances where the longest 256-row tile would outlast
// the average load of a CU. D is the head dimension (128 or 256); GATE
// applies the sigmoid output gate.
template <int W, int D, bool GATE, int KG = 1>
__global__ __launch_bounds__(W * KG * kWave) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_prefill_kernel(const FlashArgs a) {
  static_assert(KG == 1 || (KG == 2 && W == 4), "key groups: one, or two with 128-row blocks");
  constexpr int QT = 1;       // 32-row query tiles per wave
  constexpr int kWM = 32 * QT;
  constexpr int kBM = kWM * W;                 // query rows per block
  constexpr int NW = W * KG;                   // waves per block
  constexpr int kStages = W == 8 ? 3 : 2;      // loads run kStages - 1 steps ahead
  constexpr int kTK = kBN * KG;                // keys per step (one tile per key group)
  constexpr int kRowsPerWave = kTK / NW;       // K and V rows each wave moves per step
  constexpr int kKPitch = D;                   // elements: rows are unpadded, chunks swizzled
  constexpr int kVPitch = D;
  constexpr int kRowBytes = 2 * D;
  constexpr int kCPR = D / 8;                  // 16-byte chunks per row
  constexpr int kRPI = kWave / kCPR;           // rows one 1 KB DMA instruction fills
  constexpr int kInstr = kRowsPerWave / kRPI;  // DMA instructions per wave per tile, for K and for V
  static_assert(kRowsPerWave % kRPI == 0, "a wave's rows fill whole DMA instructions");
  constexpr int kTileVm = 2 * kInstr;          // DMA instructions per wave per tile
  constexpr int kWaitStep = waitcnt_vm(kStages == 3 ? kTileVm : 0);
  constexpr int kDT = D / 32;                  // 32-dim output tiles
  constexpr int kST = D / 16;                  // 16-dim score k-steps
  // K operand reads and V^T operand pairs in flight ahead of their MFMAs:
  // 4 and 3, or 3 and 2 where the 128-row, head_dim-256 block would otherwise
  // spill (its four DMA instructions per tile leave no room for more)
  constexpr bool kTight = W == 4 && D == 256;
  constexpr int kKPF = kTight ? 3 : 4;
  constexpr int kVPF = kTight ? 2 : 3;
  // one LDS object per ring stage, indexed only by compile-time stage numbers
  __shared__ __attribute__((aligned(1024))) uint16_t ks0[kTK][kKPitch];
  __shared__ __attribute__((aligned(1024))) uint16_t ks1[kTK][kKPitch];
  __shared__ __attribute__((aligned(1024))) uint16_t ks2[kStages == 3 ? kTK : 1][kKPitch];
  __shared__ __attribute__((aligned(1024))) uint16_t vs0[kTK][kVPitch];
  __shared__ __attribute__((aligned(1024))) uint16_t vs1[kTK][kVPitch];
  __shared__ __attribute__((aligned(1024))) uint16_t vs2[kStages == 3 ? kTK : 1][kVPitch];
  // each key group's running max and sum per lane, for the final merge
  __shared__ float ml_part[KG == 2 ? 2 : 1][KG == 2 ? NW : 1][kWave];
  // (with two key groups the staging rows live in the stage buffers instead)
  __shared__ __attribute__((aligned(16))) uint16_t ebuf[KG == 2 ? 1 : W][kWM][kEpiPitch];
  auto kbuf = [&](auto b) __attribute__((always_inline)) -> uint16_t(*)[kKPitch] {
    if constexpr (decltype(b)::value == 0) return ks0;
    else if constexpr (decltype(b)::value == 1) return ks1;
    else return ks2;
  };
  auto vbuf = [&](auto b) __attribute__((always_inline)) -> uint16_t(*)[kVPitch] {
    if constexpr (decltype(b)::value == 0) return vs0;
    else if constexpr (decltype(b)::value == 1) return vs1;
    else return vs2;
  };

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int rw = wid % W;        // the wave's 32 query rows within the block
  const int kgi = wid / W;       // its key group: key tiles kgi, kgi + KG, ...
  const int n32 = lane & 31;
  const int kg = lane >> 5;
  const int N = a.N;
  // Work order. Consecutive block ids are dispatched round-robin over the 8
  // XCDs (each with its own L2); XCD x takes a run of consecutive heads --
  // heads of one key/value group when the counts divide evenly -- so each L2
  // holds one group's K and V, and within an XCD the longest query tiles go
  // first. blockIdx.y is the sequence.
  const int nqt = (N + kBM - 1) / kBM;
  int h, qt;
  if (a.xcd_heads > 0) {
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    h = x * a.xcd_heads + slot % a.xcd_heads;
    qt = nqt - 1 - slot / a.xcd_heads;
  } else {
    h = blockIdx.x % a.HQ;
    qt = nqt - 1 - blockIdx.x / a.HQ;
  }
  const int b = blockIdx.y;
  const int g = h / (a.HQ / a.HKV);
  const uint16_t* kseq = a.k + b * a.k_bs + g * a.k_hs;
  const uint16_t* vseq = a.v + b * a.v_bs + g * a.v_hs;
  const int q0 = qt * kBM + rw * kWM;           // the wave's first query row
  // key tiles the block walks: up to its last row, and no tile wholly past N;
  // a step brings KG consecutive tiles
  const int kend = min((qt + 1) * kBM, N);
  const int ntiles = (kend + kBN - 1) / kBN;
  const int nsteps = (ntiles + KG - 1) / KG;
  const int my_last = min((q0 + kWM - 1) / kBN, ntiles - 1);   // the wave's last tile with a visible key

  // Direct global -> LDS tile loads, 1 KB per instruction: the 64 lanes fill
  // kRPI whole rows (lane l: row l / kCPR, physical chunk l % kCPR). Rows are
  // unpadded; a row's 16-byte chunks are XOR-swizzled so that the operand
  // reads below hit distinct banks -- K row r keeps logical chunk c at
  // physical chunk c ^ (r & 15), V row r at c ^ 4 (r & 3) -- so each lane
  // fetches the logical chunk its physical slot holds. Wave w moves rows
  // R w .. R w + R - 1 of K and of V (R = 32 / W). Rows past N repeat row
  // N - 1 (only rows past N see them, and those rows are not stored). Every
  // step issues exactly one step's loads (past the last step it reloads the
  // last step into a free stage, where nothing reads it), so the number of
  // loads in flight behind step ks is constant and so is every wait count.
  // Stage row j holds key kTK ks + j: tile KG ks + j / 32, whose rows keep the
  // same swizzle as a one-tile stage (32 is a multiple of 16).
  const int dma_row = lane / kCPR, dma_chunk = lane % kCPR;
  auto load_tile = [&](int ks, auto bs) __attribute__((always_inline)) {
    ks = ks < nsteps ? ks : nsteps - 1;
    uint16_t(*kb)[kKPitch] = kbuf(bs);
    uint16_t(*vb)[kVPitch] = vbuf(bs);
#pragma unroll
    for (int i = 0; i < kInstr; ++i) {
      const int t0 = kRowsPerWave * wid + kRPI * i;     // first stage row of this instruction
      const int trow = t0 + dma_row;
      const size_t r = static_cast<size_t>(min(ks * kTK + trow, N - 1));
      lds_dma16(kseq + r * a.k_rs + 8 * (dma_chunk ^ (trow & 15)), lds_offset(&kb[t0][0]));
      lds_dma16(vseq + r * a.v_rs + 8 * (dma_chunk ^ (4 * (trow & 3))), lds_offset(&vb[t0][0]));
    }
  };

  // Q^T operands, resident: q-tile t, lane (query q0 + 32t + n32, k-group kg)
  // holds Q[.][16 st + 8 kg .. +7]; rows past N read row N - 1
  uint4 qop[QT][kST];
  if constexpr (KG == 2) {
    // The two key groups hold the same 128 query rows: they come once, by DMA
    // into the second stage (free until step 0's barrier refills it), rows
    // 0..63 in ks1 and 64..127 in vs1, each row's chunks swizzled like a K row
    // (logical chunk c at c ^ (r & 15)), with the first tile in flight behind
    // them; every wave then reads its Q^T operands from there, conflict-free
    // like the K operand reads.
    constexpr int kQRowsPerWave = kBM / NW;               // 16
    constexpr int kQInstr = kQRowsPerWave / kRPI;         // 8 DMA instructions per wave
    static_assert(kBM == 2 * kTK && kQRowsPerWave % kRPI == 0, "the query rows fill the second stage");
#pragma unroll
    for (int i = 0; i < kQInstr; ++i) {
      const int r0 = kQRowsPerWave * wid + kRPI * i;     // first block row of this instruction
      const int qr = r0 + dma_row;
      const size_t qn = static_cast<size_t>(min(qt * kBM + qr, N - 1));
      uint16_t(*qb)[kKPitch] = r0 < kTK ? ks1 : vs1;
      lds_dma16(a.q + b * a.q_bs + qn * a.q_rs + h * a.q_hs + 8 * (dma_chunk ^ (qr & 15)),
                lds_offset(&qb[r0 % kTK][0]));
    }
    load_tile(0, IC<0>{});
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kTileVm));   // this wave's query rows landed (loads complete in order)
    lds_barrier();                                     // and every other wave's
    const int qr = rw * kWM + n32;                     // block row of this lane's query
    const char* qbase = reinterpret_cast<const char*>(qr < kTK ? &ks1[qr][0] : &vs1[qr - kTK][0]);
#pragma unroll
    for (int st = 0; st < kST; ++st)
      qop[0][st] = *reinterpret_cast<const uint4*>(qbase + 16 * ((2 * st + kg) ^ (qr & 15)));
    // the reads are complete before any wave passes step 0's barrier and refills the stage
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  } else {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const size_t qn = static_cast<size_t>(min(q0 + 32 * t + n32, N - 1));
      const uint16_t* qrow = a.q + b * a.q_bs + qn * a.q_rs + h * a.q_hs + 8 * kg;
#pragma unroll
      for (int st = 0; st < kST; ++st) qop[t][st] = ld16(qrow + 16 * st);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);   // Q is in; from here on only tile loads are in flight
    load_tile(0, IC<0>{});
    if constexpr (kStages == 3) load_tile(1, IC<1>{});
  }

  f32x16 o[kDT][QT];   // O^T: value dims 32 dt + ..., queries q0 + 32 t + n32
#pragma unroll
  for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][t][e] = 0.f;
  // Running row max (log2 units). It is only raised when some row's tile max
  // passes it by more than kSlack, so the weights exp2(s - m) stay <= 2^kSlack
  // (exact in f32, in range for bf16) and O is rescaled rarely; the final
  // o / l is the same softmax.
  constexpr float kSlack = 8.0f;
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    m_run[t] = -INFINITY;
    l_run[t] = 0.f;
  }

  const int L = lane & 15;
  const int half16 = (lane >> 4) & 1;
  // Swizzled operand addresses: one per-lane base plus an immediate. K: lane
  // (key n32, k-group kg) reads logical chunk 2 st + kg of row n32, physical
  // (2 st + kg) ^ s with s = n32 & 15, i.e. byte 32 (st ^ (s >> 1)) + 16 (kg ^ (s & 1))
  // -- 256 (st >> 3) an immediate. V: the
  // transpose read of rows 4 kg + L / 4 (+ 8, + 16 ks2) at chunk
  // 2 half16 + (L & 3) / 2 + 4 dt, physical ... + 4 (dt ^ q) with q = (L / 4) & 3
  // -- the swizzle bits (5-7 for K, 6-7 for V) are zero in the rest of the
  // lane's base, so each address is that base XOR a compile-time constant.
  // (plus the wave's key group's 32-row half of the stage)
  const int k_base = (32 * kgi + n32) * kRowBytes + 16 * (kg ^ (n32 & 1)) + 32 * ((n32 & 15) >> 1);
  const int v_base = (32 * kgi + 4 * kg + (L >> 2)) * kRowBytes + 16 * (2 * half16 + ((L & 3) >> 1)) + 8 * (L & 1) +
                     64 * ((L >> 2) & 3);
  // One key tile in ring stage `bs`. The block barrier is a bare s_barrier
  // between compiler fences: each wave first waits for its own loads of tile
  // kt (the only ones in flight), and its reads of the stage being refilled --
  // tile kt - 1's -- were consumed by MFMAs of the previous step before it
  // arrives.
  auto step = [&](int ks, auto bs) __attribute__((always_inline)) {
    constexpr int B = decltype(bs)::value;
    __builtin_amdgcn_s_waitcnt(kWaitStep);   // step ks landed; with three stages step ks + 1 may fly
    block_barrier();
    load_tile(ks + kStages - 1, IC<(B + kStages - 1) % kStages>{});   // into the stage of step ks - 1
    const int kt = KG * ks + kgi;            // this wave's key tile
    uint16_t(*kb)[kKPitch] = kbuf(bs);
    uint16_t(*vb)[kVPitch] = vbuf(bs);

    if (kt <= my_last) {   // wave-uniform: later tiles hold no key this wave sees
      // S^T = K . Q^T: element e = 4j + r is key 32 kt + 8j + 4kg + r,
      // query q0 + 32 t + n32
      f32x16 s[QT];
#pragma unroll
      for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[t][e] = 0.f;
      // K operands stream through a ring of kKPF registers: the read for
      // k-step st + kKPF is issued behind the MFMA of k-step st
      const char* kbytes = reinterpret_cast<const char*>(&kb[0][0]);
      // opaque per tile: the XORs below are recomputed, not hoisted into a
      // register per k-step (which would not fit beside the accumulators)
      int kx = k_base;
      asm volatile("" : "+v"(kx));
      auto kld = [&](int st) __attribute__((always_inline)) {
        return *reinterpret_cast<const uint4*>(kbytes + (kx ^ (32 * (st & 7))) + 256 * (st >> 3));
      };
      uint4 kq[kKPF];
#pragma unroll
      for (int i = 0; i < kKPF; ++i) kq[i] = kld(i);
#pragma unroll
      for (int st = 0; st < kST; ++st) {
        const uint4 kop = kq[st % kKPF];
        if (st + kKPF < kST) kq[st % kKPF] = kld(st + kKPF);
#pragma unroll
        for (int t = 0; t < QT; ++t)
          s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(kop), as_bf8(qop[t][st]), s[t], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kKPF, 0);
#pragma unroll
      for (int st = 0; st < kST; ++st) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, QT, 0);
        if (st + kKPF < kST) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
      // online softmax per query tile (the scale is folded into exp2's argument)
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const int qrow0 = q0 + 32 * t;
        if (kt * kBN + kBN - 1 > qrow0) {   // tile reaches past this query tile's first row
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kk = kt * kBN + 8 * (e >> 2) + 4 * kg + (e & 3);
            s[t][e] = kk > qrow0 + n32 ? -INFINITY : s[t][e];
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[t][e]);
        mx = fmaxf(mx, xor_lane<32>(mx, lane)) * a.scale_log2;
        if (__builtin_amdgcn_ballot_w64(mx > m_run[t] + kSlack) != 0) {
          const float m_new = fmaxf(m_run[t], mx);
          const float alpha = m_run[t] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[t] - m_new);
          l_run[t] *= alpha;
#pragma unroll
          for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[dt][t][e] *= alpha;
          m_run[t] = m_new;
        }
      }
      // O^T += V^T . P^T: k-step ks2 takes keys 16 ks2 + {4kg + r, 8 + 4kg + r}
      // = score elements 8 ks2 + r, 8 ks2 + 4 + r; each V^T operand serves
      // every query tile
      const char* vbytes = reinterpret_cast<const char*>(&vb[0][0]);
      int vx = v_base;
      asm volatile("" : "+v"(vx));
      uint4 pop[2][QT];
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int t = 0; t < QT; ++t) {
          float p[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            p[i] = __builtin_amdgcn_exp2f(fmaf(s[t][8 * ks2 + i], a.scale_log2, -m_run[t]));
            l_run[t] += p[i];
          }
          pop[ks2][t] = pack8(p);
        }
      // V^T operands, pair i = (ks2, dt) = (i / kDT, i % kDT), stream through a
      // ring of kVPF register pairs like the K operands
      constexpr int kNPV = 2 * kDT;
      auto vld = [&](int i, uint2* dst) __attribute__((always_inline)) {
        const int ks2 = i / kDT, dt = i % kDT;
        const char* p = vbytes + (vx ^ (64 * (dt & 3))) + 256 * (dt >> 2) + 16 * ks2 * kRowBytes;
        dst[0] = ld_tr(reinterpret_cast<const uint16_t*>(p));
        dst[1] = ld_tr(reinterpret_cast<const uint16_t*>(p + 8 * kRowBytes));
      };
      uint2 vq[kVPF][2];
#pragma unroll
      for (int i = 0; i < kVPF; ++i) vld(i, vq[i]);
#pragma unroll
      for (int i = 0; i < kNPV; ++i) {
        const uint4 vop = make_uint4(vq[i % kVPF][0].x, vq[i % kVPF][0].y, vq[i % kVPF][1].x, vq[i % kVPF][1].y);
        if (i + kVPF < kNPV) vld(i + kVPF, vq[i % kVPF]);
        const int ks2 = i / kDT, dt = i % kDT;
#pragma unroll
        for (int t = 0; t < QT; ++t)
          o[dt][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(vop), as_bf8(pop[ks2][t]), o[dt][t], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kVPF, 0);
#pragma unroll
      for (int i = 0; i < kNPV; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, QT, 0);
        if (i + kVPF < kNPV) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
    }
  };
  for (int ks = 0; ks < nsteps; ks += kStages) {
    step(ks, IC<0>{});
    if (ks + 1 < nsteps) step(ks + 1, IC<1>{});
    if constexpr (kStages == 3)
      if (ks + 2 < nsteps) step(ks + 2, IC<2>{});
  }
  // no load may still be writing this block's LDS when the block ends
  __builtin_amdgcn_s_waitcnt(kWaitVm0);

  // epilogue: element e = 4j + r of o[dt][0] is value dim 32 dt + 8j + 4kg + r
  // of query q0 + n32. out = bf16(bf16(o / l) * bf16(sigmoid(gate))) with the
  // gate, bf16(o / l) without, in passes of kEpiDims dims through this wave's
  // staging rows: bf16(o / l) into LDS, then 16-byte pieces of whole rows --
  // piece p of a pass is row p / 8, dims 8 (p % 8) .. + 7 of the pass -- for
  // the gate (its loads issued first: it does not depend on O) and the output.
  // Rows past N are not stored. With two key groups the wave pair (rw, 0),
  // (rw, 1) first merges symmetrically: wave (rw, g) keeps value dims
  // D/2 g .. D/2 g + D/2 - 1 and hands its partner the other half of its
  // output with its (max, sum), through the stage buffers (every wave is past
  // its last operand read); each rescales both to the joint max and adds them,
  // group 0's term first, so both waves hold the same sums; then each wave
  // stores its half. A group that saw no key has max -inf and contributes
  // nothing. A half is D/2 f32 per lane, written lane-fastest in 16-byte
  // pieces (each instruction 1 KB contiguous).
  static_assert(QT == 1 && D % (2 * kEpiDims) == 0, "one 32-row query tile per wave, whole passes per half");
  constexpr int kPieces = kWM * kEpiDims / 8 / kWave;   // 16-byte pieces per lane per pass
  constexpr int kDTP = kEpiDims / 32;                   // 32-dim output tiles per pass
  uint16_t(*eb)[kEpiPitch] = ebuf[KG == 2 ? 0 : rw];
  // G: the half of the value dims this wave stores (-1: all of them)
  auto finish = [&](auto gc) __attribute__((always_inline)) {
    constexpr int G = decltype(gc)::value;
    constexpr int kP0 = G < 0 ? 0 : G * (D / kEpiDims / 2);
    constexpr int kP1 = G < 0 ? D / kEpiDims : kP0 + D / kEpiDims / 2;
    uint4 gp[GATE ? kP1 - kP0 : 1][kPieces];
    if constexpr (GATE) {
#pragma unroll
      for (int c = kP0; c < kP1; ++c)
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
          const int pc = i * kWave + lane, row = pc / (kEpiDims / 8);
          const size_t qn = static_cast<size_t>(min(q0 + row, N - 1));
          gp[c - kP0][i] = *reinterpret_cast<const uint4*>(a.gate + b * a.g_bs + qn * a.g_rs + h * a.g_hs +
                                                           kEpiDims * c + 8 * (pc % (kEpiDims / 8)));
        }
    }
    if constexpr (G >= 0) {
      constexpr int kHalf = kDT / 2;
      constexpr int kT0 = G * kHalf, kO0 = (1 - G) * kHalf;   // own and partner's first output tile
      lds_barrier();
      float4* part = reinterpret_cast<float4*>(rw == 0 ? &ks0[0][0] : rw == 1 ? &ks1[0][0] : rw == 2 ? &vs0[0][0]
                                                                                                   : &vs1[0][0]);
      // slot g of the pair's buffer: the half that wave (rw, g) hands over
#pragma unroll
      for (int u = 0; u < kHalf; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          part[((G * kHalf + u) * 4 + j) * kWave + lane] =
              make_float4(o[kO0 + u][0][4 * j], o[kO0 + u][0][4 * j + 1], o[kO0 + u][0][4 * j + 2],
                          o[kO0 + u][0][4 * j + 3]);
      ml_part[0][rw + W * G][lane] = m_run[0];
      ml_part[1][rw + W * G][lane] = l_run[0];
      lds_barrier();
      const float mo = ml_part[0][rw + W * (1 - G)][lane], lo = ml_part[1][rw + W * (1 - G)][lane];
      const float mj = fmaxf(m_run[0], mo);
      const float as = m_run[0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[0] - mj);
      const float ao = mo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - mj);
      // group 0's term first
      const float a0 = G == 0 ? as : ao, a1 = G == 0 ? ao : as;
      const float l0 = G == 0 ? l_run[0] : lo, l1 = G == 0 ? lo : l_run[0];
      l_run[0] = l0 * a0 + l1 * a1;
#pragma unroll
      for (int u = 0; u < kHalf; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 p = part[(((1 - G) * kHalf + u) * 4 + j) * kWave + lane];
          const float pv[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float own = o[kT0 + u][0][4 * j + r];
            const float v0 = G == 0 ? own : pv[r], v1 = G == 0 ? pv[r] : own;
            o[kT0 + u][0][4 * j + r] = v0 * a0 + v1 * a1;
          }
        }
      // every wave has read its partner's half: the pair's stage buffer holds
      // the two waves' staging rows from here on
      lds_barrier();
      static_assert(2 * kWM * kEpiPitch * 2 <= kTK * kKPitch * 2, "two waves' staging rows fit a stage buffer");
      eb = reinterpret_cast<uint16_t(*)[kEpiPitch]>(reinterpret_cast<char*>(part) + G * kWM * kEpiPitch * 2);
    }
    const float inv = 1.0f / (l_run[0] + xor_lane<32>(l_run[0], lane));
#pragma unroll
    for (int c = kP0; c < kP1; ++c) {
#pragma unroll
      for (int u = 0; u < kDTP; ++u) {
        const int dt = kDTP * c + u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float y[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = o[dt][0][4 * j + r] * inv;
          *reinterpret_cast<uint2*>(&eb[n32][32 * u + 8 * j + 4 * kg]) =
              make_uint2(pack_bf(y[0], y[1]), pack_bf(y[2], y[3]));
        }
      }
      wave_lds_sync();
#pragma unroll
      for (int i = 0; i < kPieces; ++i) {
        const int pc = i * kWave + lane, row = pc / (kEpiDims / 8), ch = pc % (kEpiDims / 8);
        const uint4 yv = *reinterpret_cast<const uint4*>(&eb[row][8 * ch]);
        uint4 ov = yv;
        if constexpr (GATE) {
          float yf[8], gf[8];
          unpack8(yv, yf);
          unpack8(gp[c - kP0][i], gf);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float sg =
                round_bf(__builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gf[e] * 1.4426950408889634f)));
            yf[e] = round_bf(yf[e] * sg);
          }
          ov = pack8(yf);
        }
        const int qn = q0 + row;
        if (qn < N)
          *reinterpret_cast<uint4*>(a.out + b * a.o_bs + static_cast<size_t>(qn) * a.o_rs + h * D + kEpiDims * c +
                                    8 * ch) = ov;
      }
      wave_lds_sync();   // this pass's reads are done before the next pass's writes
    }
  };
  if constexpr (KG == 2) {
    if (kgi == 0) finish(IC<0>{});
    else finish(IC<1>{});
  } else {
    finish(IC<-1>{});
  }
}

// XCD-grouped order when every XCD gets whole heads of a single group
int xcd_heads(int64_t heads, int64_t kv_heads) {
  const int64_t per = heads / 8, group = heads / kv_heads;
  return (heads % 8 == 0 && per >= 1 && (group % per == 0 || per % group == 0)) ? (int)per : 0;
}

// 256-row blocks when they still give every CU a block, else 128-row blocks.
// (64- and 32-row blocks were measured slower on short prompts: a block walks
// its key tiles one after another with one tile of look-ahead, so thinner
// blocks only add more serial walks of the same latency.)
//
// Below that, head_dim 256 takes the 128-row blocks with the keys split over two
// wave groups: 8 waves and 133 KB of LDS, one block per CU (24 heads x 1024
// tokens: 43.5 -> 41 us; x 2048: 86.5 -> 80.5 us against 4 waves per block).
// At 4096 and 8192 tokens the 256-row blocks stay faster (211 against 236 us,
// 751 against 822 us), and head_dim 128 (the decode model's prompt prefill)
// measured the same either way, so it keeps its one key group.
template <int D, bool GATE>
int launch_flash(const FlashArgs& a, int64_t batch, hipStream_t stream, const char* name) {
  const int64_t t256 = (a.N + 255) / 256, t128 = (a.N + 127) / 128;
  if (a.HQ * t256 * batch >= 256)
    flash_prefill_kernel<8, D, GATE><<<dim3((unsigned)(a.HQ * t256), (unsigned)batch), 8 * kWave, 0, stream>>>(a);
  else if constexpr (D == 256)
    flash_prefill_kernel<4, D, GATE, 2><<<dim3((unsigned)(a.HQ * t128), (unsigned)batch), 8 * kWave, 0, stream>>>(a);
  else
    flash_prefill_kernel<4, D, GATE><<<dim3((unsigned)(a.HQ * t128), (unsigned)batch), 4 * kWave, 0, stream>>>(a);
  return launched(name);
}

}  // namespace

extern "C" {

int tfa_prefill_attention(const void* q, int64_t q_rs, int64_t q_hs, const void* k, int64_t k_rs, int64_t k_hs,
                          const void* v, int64_t v_rs, int64_t v_hs, const void* gate, int64_t g_rs,
                          int64_t g_hs, void* out, int64_t o_rs, int64_t n, int64_t heads, int64_t kv_heads,
                          int64_t head_dim, float scale, hipStream_t stream) {
  TFA_NONNULL(q);
  TFA_NONNULL(k);
  TFA_NONNULL(v);
  TFA_NONNULL(gate);
  TFA_NONNULL(out);
  TFA_REQUIRE(head_dim == 256, TFA_ERR_SHAPE, "tfa_prefill_attention: head_dim %lld, only 256 supported", (long long)head_dim);
  TFA_REQUIRE(n >= 128 && n % 128 == 0 && n <= (1 << 20), TFA_ERR_SHAPE,
              "tfa_prefill_attention: n %lld must be a positive multiple of %d", (long long)n, 128);
  TFA_REQUIRE(kv_heads >= 1 && heads >= kv_heads && heads % kv_heads == 0 && heads <= 65535, TFA_ERR_SHAPE,
              "tfa_prefill_attention: heads %lld not a multiple of kv_heads %lld", (long long)heads, (long long)kv_heads);
  TFA_REQUIRE(q_rs % 8 == 0 && q_hs % 8 == 0 && k_rs % 8 == 0 && k_hs % 8 == 0 && v_rs % 8 == 0 &&
                  v_hs % 8 == 0 && g_rs % 8 == 0 && g_hs % 8 == 0 && o_rs % 8 == 0,
              TFA_ERR_ALIGN, "tfa_prefill_attention: row / head strides must keep 16-byte alignment");
  TFA_ALIGN16(q);
  TFA_ALIGN16(k);
  TFA_ALIGN16(v);
  TFA_ALIGN16(gate);
  TFA_ALIGN16(out);
  FlashArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.gate = static_cast<const uint16_t*>(gate);
  a.out = static_cast<uint16_t*>(out);
  a.q_rs = (int)q_rs; a.q_hs = (int)q_hs;
  a.k_rs = (int)k_rs; a.k_hs = (int)k_hs;
  a.v_rs = (int)v_rs; a.v_hs = (int)v_hs;
  a.g_rs = (int)g_rs; a.g_hs = (int)g_hs;
  a.o_rs = (int)o_rs;
  a.N = (int)n;
  a.HQ = (int)heads;
  a.HKV = (int)kv_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.xcd_heads = xcd_heads(heads, kv_heads);
  return launch_flash<256, true>(a, 1, stream, "flash_prefill");
}

int tfa_causal_attention(const void* q, int64_t q_rs, int64_t q_hs, int64_t q_bs, const void* k, int64_t k_rs,
                         int64_t k_hs, int64_t k_bs, const void* v, int64_t v_rs, int64_t v_hs, int64_t v_bs,
                         void* out, int64_t o_rs, int64_t o_bs, int64_t batch, int64_t n, int64_t heads,
                         int64_t kv_heads, int64_t head_dim, float scale, hipStream_t stream) {
  TFA_NONNULL(q);
  TFA_NONNULL(k);
  TFA_NONNULL(v);
  TFA_NONNULL(out);
  TFA_REQUIRE(head_dim == 128 || head_dim == 256, TFA_ERR_SHAPE,
              "tfa_causal_attention: head_dim %lld not in {128, 256}", (long long)head_dim);
  TFA_REQUIRE(n >= 1 && n <= (1 << 20), TFA_ERR_SHAPE, "tfa_causal_attention: n %lld not in [1, 2^20]", (long long)n);
  TFA_REQUIRE(batch >= 1 && batch <= 65535, TFA_ERR_SHAPE, "tfa_causal_attention: batch %lld out of range",
              (long long)batch);
  TFA_REQUIRE(kv_heads >= 1 && heads >= kv_heads && heads % kv_heads == 0 && heads <= 65535, TFA_ERR_SHAPE,
              "tfa_causal_attention: heads %lld not a multiple of kv_heads %lld", (long long)heads, (long long)kv_heads);
  const int64_t lim = int64_t(1) << 31;
  TFA_REQUIRE(q_rs >= 0 && q_rs < lim && k_rs >= 0 && k_rs < lim && v_rs >= 0 && v_rs < lim && o_rs >= 0 &&
                  o_rs < lim && q_hs >= 0 && q_hs < lim && k_hs >= 0 && k_hs < lim && v_hs >= 0 && v_hs < lim &&
                  q_bs >= 0 && k_bs >= 0 && v_bs >= 0 && o_bs >= 0,
              TFA_ERR_SHAPE, "tfa_causal_attention: strides must be non-negative, row / head strides below 2^31");
  TFA_REQUIRE(q_rs % 8 == 0 && q_hs % 8 == 0 && q_bs % 8 == 0 && k_rs % 8 == 0 && k_hs % 8 == 0 && k_bs % 8 == 0 &&
                  v_rs % 8 == 0 && v_hs % 8 == 0 && v_bs % 8 == 0 && o_rs % 8 == 0 && o_bs % 8 == 0,
              TFA_ERR_ALIGN, "tfa_causal_attention: strides must keep 16-byte alignment");
  TFA_ALIGN16(q);
  TFA_ALIGN16(k);
  TFA_ALIGN16(v);
  TFA_ALIGN16(out);
  FlashArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.out = static_cast<uint16_t*>(out);
  a.q_bs = q_bs; a.k_bs = k_bs; a.v_bs = v_bs; a.o_bs = o_bs;
  a.q_rs = (int)q_rs; a.q_hs = (int)q_hs;
  a.k_rs = (int)k_rs; a.k_hs = (int)k_hs;
  a.v_rs = (int)v_rs; a.v_hs = (int)v_hs;
  a.o_rs = (int)o_rs;
  a.N = (int)n;
  a.HQ = (int)heads;
  a.HKV = (int)kv_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.xcd_heads = xcd_heads(heads, kv_heads);
  if (head_dim == 128) return launch_flash<128, false>(a, batch, stream, "causal_attention");
  return launch_flash<256, false>(a, batch, stream, "causal_attention");
}

}  // extern "C"
