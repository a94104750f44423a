// Shared device helpers for the gfx950 kernels: bf16 bit conversions, 128-bit
// vector access, wave64 reductions and the "last block finishes" handshake.
//
// Every kernel in this library stores bf16 as raw uint16_t bits. Conversion
// from f32 is round-to-nearest-even, the rounding torch's `.to(bfloat16)`
// performs, so a value computed in f32 lands on the same bf16 the oracle's
// torch spelling would produce from the same f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#define TFA_DEV __device__ __forceinline__

namespace tfa {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 bits
TFA_DEV float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// f32 -> bf16 on gfx950's v_cvt_pk_bf16_f32: round to nearest even (the rule
// torch's c10::BFloat16 applies to finite values), two values per instruction.
typedef float tfa_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 tfa_bf16x2 __attribute__((ext_vector_type(2)));
TFA_DEV uint32_t pack_bf(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(tfa_f32x2{lo, hi}, tfa_bf16x2));
}
TFA_DEV uint32_t f2bf(float f) { return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f))); }

// bf16 round trip: the value f takes after landing in bf16.
TFA_DEV float round_bf(float f) { return bf2f(f2bf(f)); }

// low / high bf16 of a packed 32-bit word, as f32
TFA_DEV float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
TFA_DEV float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }


// 8 bf16 (one 16-byte vector) <-> 8 floats
TFA_DEV void unpack8(const uint4 v, float* f) {
  f[0] = lo_bf(v.x); f[1] = hi_bf(v.x);
  f[2] = lo_bf(v.y); f[3] = hi_bf(v.y);
  f[4] = lo_bf(v.z); f[5] = hi_bf(v.z);
  f[6] = lo_bf(v.w); f[7] = hi_bf(v.w);
}

TFA_DEV uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf(f[0], f[1]);
  v.y = pack_bf(f[2], f[3]);
  v.z = pack_bf(f[4], f[5]);
  v.w = pack_bf(f[6], f[7]);
  return v;
}

// a.lo * b.lo + a.hi * b.hi + c over packed bf16 pairs (v_dot2_f32_bf16; a
// bf16 x bf16 product is exact in f32)
TFA_DEV float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

TFA_DEV uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Streaming load for data read exactly once (weights, KV cache): non-temporal
// hint so it does not evict reusable lines from L2 / MALL.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
TFA_DEV uint4 ld16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
TFA_DEV void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
// Streaming store for outputs no kernel of this launch reads back and the next
// does not read straight from L2 (many-row passes): non-temporal hint.
TFA_DEV void st16_stream(void* p, uint4 v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------- reductions

// Max over each 16-lane row of the wave (every lane gets its row's max) by DPP
// lane permutations -- quad swaps, then the half-row and row mirrors -- with
// no LDS traffic.
template <int CTRL>
TFA_DEV float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
TFA_DEV float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));    // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp_f32<0x4E>(v));    // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp_f32<0x141>(v));   // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));   // row_mirror
  return v;
}
// Sum over each 16-lane row the same way: quads first, then the half-row and
// row mirrors; every lane of the row ends with the identical value.
TFA_DEV float row16_sum(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return v;
}

// Max / sum over the four 16-lane rows (lanes l, l ^ 16, l ^ 32, l ^ 48) with
// gfx950's row swaps: permlane32_swap pairs lane l with l ^ 32, then
// permlane16_swap pairs l with l ^ 16 -- no LDS round trip.
TFA_DEV float rows4_max(float v) {
  auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
  auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(y[0]), __uint_as_float(y[1]));
}
TFA_DEV float rows4_sum(float v) {
  auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(y[0]) + __uint_as_float(y[1]);
}

// Sum / max over the lanes that differ from this one only in the low K bits of
// the lane id (K <= 6), bottom up: quad swaps (bits 0, 1), the half-row and row
// mirrors (bits 2, 3 -- once the smaller groups are uniform, a mirror partner
// holds the other group's value), then the row swaps (bits 4, 5). No step goes
// through LDS, and every lane of a group ends with the identical value.
template <int K>
TFA_DEV float lanes_sum(float v) {
  if (K >= 1) v += dpp_f32<0xB1>(v);
  if (K >= 2) v += dpp_f32<0x4E>(v);
  if (K >= 3) v += dpp_f32<0x141>(v);
  if (K >= 4) v += dpp_f32<0x140>(v);
  if (K >= 5) {
    auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(y[0]) + __uint_as_float(y[1]);
  }
  if (K >= 6) {
    auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(x[0]) + __uint_as_float(x[1]);
  }
  return v;
}
template <int K>
TFA_DEV float lanes_max(float v) {
  if (K >= 1) v = fmaxf(v, dpp_f32<0xB1>(v));
  if (K >= 2) v = fmaxf(v, dpp_f32<0x4E>(v));
  if (K >= 3) v = fmaxf(v, dpp_f32<0x141>(v));
  if (K >= 4) v = fmaxf(v, dpp_f32<0x140>(v));
  if (K >= 5) {
    auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(y[0]), __uint_as_float(y[1]));
  }
  if (K >= 6) {
    auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
  }
  return v;
}
TFA_DEV float wave_sum(float v) { return lanes_sum<6>(v); }
TFA_DEV float wave_max(float v) { return lanes_max<6>(v); }

constexpr int log2_const(int n) { return n <= 1 ? 0 : 1 + log2_const(n / 2); }

// Multi-row wave reduction: v[0..R) are one lane's partial sums of R rows.
// Instead of R full butterflies (6R exchanges) the rows are halved at each step
// -- a lane keeps the half of the rows its mask bit selects and adds the
// partner's partials for that half -- so R = 8 costs 4+2+1+3 = 10 exchanges and
// R = 16 costs 17, each a row swap or a DPP move (no LDS). On return every
// lane holds the wave total of one row, `row = wave_rows_owner<R>(lane)`; each
// row's total is replicated on 64/R lanes.
template <int R>
TFA_DEV int wave_rows_owner(int lane) {
  int row = 0;
  int n = R;
#pragma unroll
  for (int m = 32; m >= 1 && n > 1; m >>= 1, n >>= 1)
    if (lane & m) row += n / 2;
  return row;
}

// Partner value of lane ^ M (M a power of two): row swaps for 32 and 16 are
// handled in RowHalver itself; within a 16-lane row it takes DPP moves (a row
// rotate by 8 is lane ^ 8 in either direction; lane ^ 4 is the half-row
// mirror, lane ^ 7, followed by the quad reversal, lane ^ 3).
template <int M>
TFA_DEV float xor_partner(float v, int) {
  if constexpr (M == 8) return dpp_f32<0x128>(v);   // row_ror:8
  if constexpr (M == 4) return dpp_f32<0x1B>(dpp_f32<0x141>(v));   // quad_perm [3, 2, 1, 0] of row_half_mirror
  if constexpr (M == 2) return dpp_f32<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  if constexpr (M == 1) return dpp_f32<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  return v;
}

// Value of lane ^ M for any M (float or int bits): the row swaps for 32 and 16
// (each lane keeps the half of the swapped pair that came from its partner),
// DPP within a row.
template <int M>
TFA_DEV uint32_t xor_lane_bits(uint32_t v, int lane) {
  if constexpr (M == 32) {
    auto x = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? x[0] : x[1];
  } else if constexpr (M == 16) {
    auto x = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? x[0] : x[1];
  } else {
    return __builtin_bit_cast(uint32_t, xor_partner<M>(__builtin_bit_cast(float, v), lane));
  }
}
template <int M>
TFA_DEV float xor_lane(float v, int lane) { return __uint_as_float(xor_lane_bits<M>(__float_as_uint(v), lane)); }
template <int M>
TFA_DEV int xor_lane(int v, int lane) { return static_cast<int>(xor_lane_bits<M>(static_cast<uint32_t>(v), lane)); }

template <int N, int M>
struct RowHalver {
  TFA_DEV static void run(float* v, int lane) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      if constexpr (M == 32 || M == 16) {
        // lane l keeps row j (bit clear) or j + N/2 (bit set) and adds its
        // partner's other half: a row swap returns exactly those two values
        auto x = M == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + N / 2]), false, false)
                         : __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j + N / 2]), false, false);
        v[j] = __uint_as_float(x[0]) + __uint_as_float(x[1]);
      } else {
        const bool upper = (lane & M) != 0;
        const float keep = upper ? v[j + N / 2] : v[j];
        const float send = upper ? v[j] : v[j + N / 2];
        v[j] = keep + xor_partner<M>(send, lane);
      }
    }
    RowHalver<N / 2, M / 2>::run(v, lane);
  }
};
// one row left: the full sum over lane bits M .. 0
template <int M>
struct RowHalver<1, M> {
  TFA_DEV static void run(float* v, int) { v[0] = lanes_sum<log2_const(M) + 1>(v[0]); }
};
template <>
struct RowHalver<1, 0> {
  TFA_DEV static void run(float*, int) {}
};

template <int R>
TFA_DEV float wave_sum_rows(float* v, int lane) {
  RowHalver<R, 32>::run(v, lane);
  return v[0];
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
TFA_DEV float group_sum(float v) {
  return lanes_sum<log2_const(WIDTH)>(v);
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `scratch` holds one
// float per wave. Every thread gets the total; waves are summed in wave order
// so the result does not depend on scheduling.
TFA_DEV float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  v = wave_sum(v);
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < nw; ++w) t += scratch[w];
  __syncthreads();
  return t;
}

// ------------------------------------------------------------ split-K sums
// Sum of the first `ks` (1 <= ks <= MAXKS) of p[0], p[stride], p[2 stride], ...
// in split order, with every load issued before the first add and none behind
// a branch (a split past ks re-reads split ks - 1 and a select leaves it out of
// the sum): one memory round trip, not one per split (a runtime-bounded loop,
// or a load per branch, is waited for in turn).
constexpr int kMaxSplitsK = 8;
template <int MAXKS = kMaxSplitsK>
TFA_DEV float sum_splits(const float* p, size_t stride, int ks) {
  float v[MAXKS];
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) v[s] = p[static_cast<size_t>(min(s, ks - 1)) * stride];
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) acc += s < ks ? v[s] : 0.f;
  return acc;
}

// The same for eight consecutive floats (two 16-byte loads per split);
// p 16-byte aligned, stride a multiple of 4.
template <int MAXKS = kMaxSplitsK>
TFA_DEV void sum_splits8(const float* p, size_t stride, int ks, float* acc) {
  float4 v[MAXKS][2];
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) {
    const float4* q = reinterpret_cast<const float4*>(p + static_cast<size_t>(min(s, ks - 1)) * stride);
    v[s][0] = q[0];
    v[s][1] = q[1];
  }
  __builtin_amdgcn_sched_barrier(0);   // every load out before the first add
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) {
    const bool in = s < ks;
    acc[0] += in ? v[s][0].x : 0.f; acc[1] += in ? v[s][0].y : 0.f;
    acc[2] += in ? v[s][0].z : 0.f; acc[3] += in ? v[s][0].w : 0.f;
    acc[4] += in ? v[s][1].x : 0.f; acc[5] += in ? v[s][1].y : 0.f;
    acc[6] += in ? v[s][1].z : 0.f; acc[7] += in ? v[s][1].w : 0.f;
  }
}

// 1/sqrt(x) with correctly rounded sqrt and division: the value torch's CPU
// `rsqrt` returns for the same f32 input.
TFA_DEV float rsqrt_rn(float x) { return 1.0f / __fsqrt_rn(x); }

TFA_DEV float silu(float x) { return x / (1.0f + __expf(-x)); }

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector-memory
// operations are in flight, expcnt and lgkmcnt left open. vmcnt is six bits,
// split over bits [3:0] and [15:14] of the immediate.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
static_assert(waitcnt_vm(0) == 0xF70 && waitcnt_vm(16) == 0x4F70 && waitcnt_vm(63) == 0xCF7F,
              "vmcnt encoding");

// Direct global -> LDS load of 16 bytes per lane: lane i's bytes land at LDS
// byte offset lds_off + 16 i (lds_off, held in M0, is wave-uniform; lanes
// switched off by exec write nothing). Issued as an instruction the compiler
// does not see into, so its wait-count bookkeeping does not make every LDS read
// wait for every such load in flight: the caller tracks these loads with its
// own vmcnt waits (vector-memory loads complete in issue order), and must wait
// for all of them before its block ends.
TFA_DEV void lds_dma16(const void* g, uint32_t lds_off) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_off) : "memory");
}
// The same for data read exactly once (a decode cache): non-temporal, as the
// streaming register loads.
TFA_DEV void lds_dma16_stream(const void* g, uint32_t lds_off) {
  asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds_off) : "memory");
}

// The 32-bit LDS byte offset of a __shared__ object.
template <typename T>
TFA_DEV uint32_t lds_offset(T* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)p));
}

// Block barrier that leaves loads in flight: the compiler may not move memory
// operations across it, and it adds no wait of its own (a __syncthreads() also
// waits for every outstanding load, which would drain a software pipeline).
// The caller waits for what the other waves must see before calling it.
TFA_DEV void block_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// s_waitcnt immediate waiting for every LDS (and scalar-memory) operation of
// the wave, vmcnt and expcnt left open.
constexpr int kWaitLgkm0 = 15 | (7 << 4) | (0 << 8) | (3 << 14);

// Block barrier for an LDS hand-off: this wave's LDS operations complete, then
// every wave meets. Loads into registers stay in flight -- the compiler waits
// for each one where it is used -- where a __syncthreads() would drain them all.
TFA_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  block_barrier();
}

// ------------------------------------------------------------ greedy pick
// (value, index) order for greedy argmax: the larger value wins, equal values go
// to the lower index (torch.argmax), NaN never wins.
TFA_DEV bool better_pick(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// The rest of a block-wide pick: each thread's (best_v, best_i) across the wave
// (row swaps / DPP, no LDS), then the waves in order through s_v / s_i (one
// entry per wave). The result is valid in thread 0.
TFA_DEV int block_best_reduce(float best_v, int best_i, float* s_v, int* s_i) {
  const int t = threadIdx.x, nt = blockDim.x;
  const int lane = t & (kWave - 1);
  auto step = [&](auto mc) __attribute__((always_inline)) {
    constexpr int M = decltype(mc)::value;
    const float ov = xor_lane<M>(best_v, lane);
    const int oi = xor_lane<M>(best_i, lane);
    if (better_pick(ov, oi, best_v, best_i)) {
      best_v = ov;
      best_i = oi;
    }
  };
  step(std::integral_constant<int, 32>{});
  step(std::integral_constant<int, 16>{});
  step(std::integral_constant<int, 8>{});
  step(std::integral_constant<int, 4>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 1>{});
  if ((t & (kWave - 1)) == 0) {
    s_v[t / kWave] = best_v;
    s_i[t / kWave] = best_i;
  }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < nt / kWave; ++w)
      if (better_pick(s_v[w], s_i[w], best_v, best_i)) {
        best_v = s_v[w];
        best_i = s_i[w];
      }
  }
  return best_i;
}

// The best (value, lowest index) pair of nb candidates, reduced by a whole block
// (blockDim.x a multiple of 64, at most 1024; s_v / s_i hold one entry per
// wave). Each thread issues eight loads before its first compare. The returned
// index is valid in thread 0.
TFA_DEV int block_best(const float* bv, const int* bi, int nb, float* s_v, int* s_i) {
  const int t = threadIdx.x, nt = blockDim.x;
  float best_v = -3.402823466e38f;
  int best_i = 0x7fffffff;
  for (int b0 = t; b0 < nb; b0 += 8 * nt) {
    float v[8];
    int ix[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int b = b0 + u * nt;
      const bool ok = b < nb;
      v[u] = ok ? bv[b] : -3.402823466e38f;
      ix[u] = ok ? bi[b] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (better_pick(v[u], ix[u], best_v, best_i)) {
        best_v = v[u];
        best_i = ix[u];
      }
  }
  return block_best_reduce(best_v, best_i, s_v, s_i);
}

// The same pick in one memory round trip for nb <= U * blockDim.x: every
// candidate load is issued at once (past nb at a clamped index, left out of the
// compare), then `between()` -- the caller's loads that must not wait behind
// these -- and only then the compares.
template <int U, typename F>
TFA_DEV int block_best_once(const float* bv, const int* bi, int nb, float* s_v, int* s_i, F&& between) {
  const int t = threadIdx.x, nt = blockDim.x;
  float v[U];
  int ix[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int b = min(t + u * nt, nb - 1);
    v[u] = bv[b];
    ix[u] = bi[b];
  }
  __builtin_amdgcn_sched_barrier(0);
  between();
  __builtin_amdgcn_sched_barrier(0);
  float best_v = -3.402823466e38f;
  int best_i = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (t + u * nt < nb && better_pick(v[u], ix[u], best_v, best_i)) {
      best_v = v[u];
      best_i = ix[u];
    }
  return block_best_reduce(best_v, best_i, s_v, s_i);
}

}  // namespace tfa
