// Causal GQA prefill attention, head_dim 256, with the output gate
// (Qwen3.5-family full-attention layer, Qwen3.8-27B shapes: 24 query heads
// over 4 key/value heads), on bf16 MFMA.
//
// One 512-thread block per (query head, 128 query rows); each pair of waves
// owns 32 query rows -- one wave per half of the head dims -- and walks the
// key tiles (32 keys) up to its diagonal. Per tile:
//
//   S^T = K . Q^T     v_mfma_f32_32x32x16_bf16, M = 32 keys, N = 32 queries;
//                     each wave of the pair reduces its 128 dims (8 k-steps,
//                     its half of Q resident as the B operand, K from LDS row
//                     reads) and the two partials are added through LDS.
//   online softmax    per query (the MFMA output column): the lane holds 16
//                     of the tile's keys, its partner lane (l ^ 32) the other
//                     16 -- one exchange for the row max; exp2 with the
//                     scale folded in; the running max is only raised (and O
//                     rescaled) when a row's max passes it by more than 2^8.
//   O^T += V^T . P^T  M = 32 value dims (4 tiles over the wave's half of D),
//                     K = 16 keys per step; P^T is the bf16 score accumulator (its key
//                     slots relabelled), V^T comes from ds_read_b64_tr_b16
//                     transpose reads of the row-major V tile.
//
// K and V tiles stream global -> LDS with global_load_lds_dwordx4 (no register
// staging), three buffers deep (loads run two tiles ahead); with the score
// exchange 138 KB of LDS per block, two waves per SIMD.
// Epilogue in the reference's order: out = bf16(bf16(o / l) * bf16(sigmoid(gate))).
//
// Reference (jingchangshi/TileFoundry): examples/qwen3_8_27b_prefill-tilelang/model.py:305-324
// (Attention.attention), kernels/attention.py:1-19,313-438 (attention_ws / attention_tir).
#include <float.h>

#include <type_traits>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int D = 256;
constexpr int kBM = 128;    // query rows per block
constexpr int kBN = 32;     // keys per tile
constexpr int kThreads = 256;
constexpr int kChunks = D / 8;   // 16-byte chunks per 512-byte row

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

TFA_DEV bf16x8 as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

struct FlashArgs {
  const uint16_t* q;     // element (n, h, d) at q + n*q_rs + h*q_hs + d
  const uint16_t* k;     // (n, g, d) at k + n*k_rs + g*k_hs + d
  const uint16_t* v;
  const uint16_t* gate;  // like q
  uint16_t* out;         // (n, h*256 + d) at out + n*o_rs + h*256 + d
  int q_rs, q_hs, k_rs, k_hs, v_rs, v_hs, g_rs, g_hs, o_rs;
  int N, HQ, HKV;
  int xcd_heads;         // heads per XCD in the work order (0: plain order)
  float scale_log2;      // head_dim^-1/2 * log2(e)
};

// LDS tiles hold one key per row. K rows are padded to 528 bytes (+4 banks per
// row): the K operand read (16 rows, one 16-byte chunk per half-wave) is
// conflict-free. V rows are padded to 576 bytes (+16 banks per row): the
// transpose reads (4 rows x 64 bytes per half-wave) are conflict-free. Every
// operand address is one per-lane base plus an immediate offset.
constexpr int kKPitch = D + 8;    // elements
constexpr int kVPitch = D + 32;
constexpr int kPairs = 4;         // wave pairs per block, 32 queries each
constexpr int kStages = 3;        // K / V tile buffers: loads run two tiles ahead
constexpr int kHalf = D / 2;      // head dims per wave of a pair

TFA_DEV uint2 ld_tr(const uint16_t* lds_elem) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_elem));
  return __builtin_bit_cast(uint2, v);
}

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) with expcnt / lgkmcnt left open.
constexpr int kWaitVm8 = 8 | (7 << 4) | (15 << 8);
constexpr int kWaitVm0 = 0 | (7 << 4) | (15 << 8);

template <int N>
using IC = std::integral_constant<int, N>;

// 512 threads: wave pair p owns queries q0 = 128 qt + 32 p; wave `half` of the
// pair owns head dims [128 half, 128 half + 128) of the scores' reduction and
// of the output. The pair's partial scores meet in LDS (f32 addition is
// commutative, so both waves hold bit-identical scores and run the same
// softmax).
__global__ __launch_bounds__(2 * kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_prefill_kernel(const FlashArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[kStages][kBN][kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kStages][kBN][kVPitch];
  __shared__ float xch[kPairs][2][16][kWave];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);   // wave-uniform, scalar
  const int pair = wid >> 1;
  const int half = wid & 1;
  const int n32 = lane & 31;    // MFMA column (query) / row (key, value dim) index
  const int kg = lane >> 5;     // k-group
  // Work order. Consecutive block ids are dispatched round-robin over the 8
  // XCDs (each with its own L2); XCD x takes a run of consecutive heads --
  // heads of one key/value group when the counts divide evenly -- so each L2
  // holds one group's K and V, and within an XCD the longest query tiles go
  // first.
  const int nqt = a.N / kBM;
  int h, qt;
  if (a.xcd_heads > 0) {
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    h = x * a.xcd_heads + slot % a.xcd_heads;
    qt = nqt - 1 - slot / a.xcd_heads;
  } else {
    h = blockIdx.x % a.HQ;
    qt = nqt - 1 - blockIdx.x / a.HQ;
  }
  const int g = h / (a.HQ / a.HKV);
  const int q0 = qt * kBM + pair * 32;         // the pair's first query row
  const int ntiles = (qt + 1) * kBM / kBN;     // key tiles the block walks
  const int my_last = q0 / kBN;                // the pair's diagonal tile

  // direct global -> LDS tile loads, one 512-byte row per instruction (lanes
  // 0..31): wave w moves rows 4w .. 4w+3 of K and of V
  // (row pointers are wave-uniform: scalar base + the lane's 16-byte offset)
  auto load_tile = [&](int kt, int buf) __attribute__((always_inline)) {
    const size_t r0 = static_cast<size_t>(kt) * kBN + 4 * wid;
    if (lane < 32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t* krow = a.k + (r0 + i) * a.k_rs + g * a.k_hs;
        const uint16_t* vrow = a.v + (r0 + i) * a.v_rs + g * a.v_hs;
        __builtin_amdgcn_global_load_lds(krow + 8 * n32,
                                         (__attribute__((address_space(3))) void*)&ks[buf][4 * wid + i][0], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vrow + 8 * n32,
                                         (__attribute__((address_space(3))) void*)&vs[buf][4 * wid + i][0], 16, 0, 0);
      }
    }
  };

  // this wave's half of Q, resident: lane (query q0 + n32, k-group kg) holds
  // Q[.][128 half + 16 st + 8 kg .. +7]
  uint4 qop[kHalf / 16];
  {
    const uint16_t* qrow = a.q + static_cast<size_t>(q0 + n32) * a.q_rs + h * a.q_hs + kHalf * half + 8 * kg;
#pragma unroll
    for (int st = 0; st < kHalf / 16; ++st) qop[st] = ld16(qrow + 16 * st);
  }
  load_tile(0, 0);
  if (ntiles > 1) load_tile(1, 1);

  f32x16 o[kHalf / 32];   // O^T rows (value dims) 128 half + 32 mt + ...
#pragma unroll
  for (int mt = 0; mt < kHalf / 32; ++mt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[mt][e] = 0.f;
  // Running row max (log2 units). It is only raised when some row's tile max
  // passes it by more than kSlack, so the weights exp2(s - m) stay <= 2^kSlack
  // (exact in f32, in range for bf16) and O is rescaled rarely; the final
  // o / l is the same softmax.
  constexpr float kSlack = 8.0f;
  float m_run = -INFINITY, l_run = 0.f;

  const int L = lane & 15;
  const int half16 = (lane >> 4) & 1;
  int buf = 0;
  for (int kt = 0; kt < ntiles; ++kt) {
    if (kt + 1 < ntiles) __builtin_amdgcn_s_waitcnt(kWaitVm8);   // tile kt landed, kt + 1 may fly
    else __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();   // tile kt visible; every wave is done with iteration kt - 1
    if (kt + 2 < ntiles) load_tile(kt + 2, buf == 0 ? 2 : buf - 1);   // the buffer of tile kt - 1

    const bool active = kt <= my_last;   // pair-uniform: later tiles hold no visible key
    f32x16 s;
    const uint16_t* vrow = &vs[buf][4 * kg + (L >> 2)][kHalf * half + 16 * half16 + 4 * (L & 3)];
    uint4 vop0[kHalf / 32], vop1[kHalf / 32];
    if (active) {
      // partial S^T = K[:, half] . Q[:, half]^T: element e = 4j + r is key
      // kt*32 + 8j + 4kg + r, query q0 + n32
      const uint16_t* krow = &ks[buf][n32][kHalf * half + 8 * kg];
      uint4 kop[kHalf / 16];
#pragma unroll
      for (int st = 0; st < kHalf / 16; ++st) kop[st] = *reinterpret_cast<const uint4*>(krow + 16 * st);
      // V^T operands of this wave's value dims (A operand, row = value dim
      // 128 half + 32 mt + n32): key rows 16 ks2 + 4kg + L/4 and +8
#pragma unroll
      for (int mt = 0; mt < kHalf / 32; ++mt) {
        const uint2 v1 = ld_tr(vrow + 32 * mt);
        const uint2 v2 = ld_tr(vrow + 8 * kVPitch + 32 * mt);
        vop0[mt] = make_uint4(v1.x, v1.y, v2.x, v2.y);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
      for (int st = 0; st < kHalf / 16; ++st)
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(kop[st]), as_bf8(qop[st]), s, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; ++e) xch[pair][half][e][lane] = s[e];
#pragma unroll
      for (int mt = 0; mt < kHalf / 32; ++mt) {
        const uint2 v1 = ld_tr(vrow + 16 * kVPitch + 32 * mt);
        const uint2 v2 = ld_tr(vrow + 24 * kVPitch + 32 * mt);
        vop1[mt] = make_uint4(v1.x, v1.y, v2.x, v2.y);
      }
    }
    __syncthreads();   // both halves of every pair's scores are in LDS

    if (active) {
      // full (unscaled) score; the scale is applied inside exp2's argument
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[e] += xch[pair][half ^ 1][e][lane];
        mx = fmaxf(mx, s[e]);
      }
      if (kt == my_last) {   // the diagonal tile: keys past the query are masked
        mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kk = 8 * (e >> 2) + 4 * kg + (e & 3);
          s[e] = kk > n32 ? -INFINITY : s[e];
          mx = fmaxf(mx, s[e]);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave)) * a.scale_log2;   // log2 units (scale > 0)
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kSlack) != 0) {   // raise the max: rescale
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int mt = 0; mt < kHalf / 32; ++mt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[mt][e] *= alpha;
        m_run = m_new;
      }
      // O^T += V^T . P^T. P^T is the B operand: k-step ks2 takes keys
      // 16ks2 + {4kg + r, 8 + 4kg + r} = score elements 8ks2 + r, 8ks2 + 4 + r
      auto pv = [&](int ks2, const uint4* vop) __attribute__((always_inline)) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          p[i] = __builtin_amdgcn_exp2f(fmaf(s[8 * ks2 + i], a.scale_log2, -m_run));   // masked: exp2(-inf) = 0
          l_run += p[i];
        }
        const uint4 pop = pack8(p);   // bf16 weights into the value product
#pragma unroll
        for (int mt = 0; mt < kHalf / 32; ++mt)
          o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(vop[mt]), as_bf8(pop), o[mt], 0, 0, 0);
      };
      pv(0, vop0);
      pv(1, vop1);
    }
    buf = buf == kStages - 1 ? 0 : buf + 1;
  }

  // epilogue: element e = 4j + r of o[mt] is value dim 128 half + 32mt + 8j + 4kg + r
  // of query q0 + n32
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  const float inv = 1.0f / l_tot;
  const size_t qn = static_cast<size_t>(q0 + n32);
  const uint16_t* grow = a.gate + qn * a.g_rs + h * a.g_hs + kHalf * half;
  uint16_t* orow = a.out + qn * a.o_rs + h * D + kHalf * half;
#pragma unroll
  for (int mt = 0; mt < kHalf / 32; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = 32 * mt + 8 * j + 4 * kg;
      const uint2 gv = *reinterpret_cast<const uint2*>(grow + d0);
      const float gx[4] = {lo_bf(gv.x), hi_bf(gv.x), lo_bf(gv.y), hi_bf(gv.y)};
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // sigmoid from the hardware exp2 / reciprocal (within 2 f32 ulps; the
        // result lands in bf16)
        const float sg = round_bf(__builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gx[r] * 1.4426950408889634f)));
        y[r] = round_bf(round_bf(o[mt][4 * j + r] * inv) * sg);
      }
      *reinterpret_cast<uint2*>(orow + d0) = make_uint2(pack_bf(y[0], y[1]), pack_bf(y[2], y[3]));
    }
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
  TFA_REQUIRE(head_dim == D, TFA_ERR_SHAPE, "tfa_prefill_attention: head_dim %lld, only 256 supported", (long long)head_dim);
  TFA_REQUIRE(n >= kBM && n % kBM == 0 && n <= (1 << 20), TFA_ERR_SHAPE,
              "tfa_prefill_attention: n %lld must be a positive multiple of %d", (long long)n, kBM);
  TFA_REQUIRE(kv_heads >= 1 && heads >= kv_heads && heads % kv_heads == 0 && heads <= 65535, TFA_ERR_SHAPE,
              "tfa_prefill_attention: heads %lld not a multiple of kv_heads %lld", (long long)heads, (long long)kv_heads);
  TFA_REQUIRE(q_rs % 8 == 0 && q_hs % 8 == 0 && k_rs % 8 == 0 && k_hs % 8 == 0 && v_rs % 8 == 0 &&
                  v_hs % 8 == 0 && g_rs % 4 == 0 && g_hs % 4 == 0 && o_rs % 4 == 0,
              TFA_ERR_ALIGN, "tfa_prefill_attention: row / head strides must keep 16-byte (q, k, v) and 8-byte (gate, out) alignment");
  TFA_ALIGN16(q);
  TFA_ALIGN16(k);
  TFA_ALIGN16(v);
  TFA_REQUIRE(aligned4(gate) && (reinterpret_cast<uintptr_t>(gate) & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
              TFA_ERR_ALIGN, "tfa_prefill_attention: gate / out must be 8-byte aligned");
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
  // XCD-grouped order when every XCD gets whole heads of a single group
  const int64_t per = heads / 8, group = heads / kv_heads;
  a.xcd_heads = (heads % 8 == 0 && per >= 1 && (group % per == 0 || per % group == 0)) ? (int)per : 0;
  flash_prefill_kernel<<<(unsigned)(heads * (n / kBM)), 2 * kThreads, 0, stream>>>(a);
  return launched("flash_prefill");
}

}  // extern "C"
