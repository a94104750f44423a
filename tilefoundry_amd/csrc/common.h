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

TFA_DEV uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Streaming load for data read exactly once (weights, KV cache): non-temporal
// hint so it does not evict reusable lines from L2 / MALL.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
TFA_DEV uint4 ld16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
TFA_DEV void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

// ---------------------------------------------------------------- reductions
TFA_DEV float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

TFA_DEV float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Multi-row wave reduction: v[0..R) are one lane's partial sums of R rows.
// Instead of R full butterflies (6R shuffles) the rows are halved at each step
// -- a lane keeps the half of the rows its mask bit selects and adds the
// partner's partials for that half -- so R = 8 costs 4+2+1+3 = 10 shuffles and
// R = 16 costs 17. On return every lane holds the wave total of one row,
// `row = wave_rows_owner<R>(lane)`; each row's total is replicated on 64/R lanes.
template <int R>
TFA_DEV int wave_rows_owner(int lane) {
  int row = 0;
  int n = R;
#pragma unroll
  for (int m = 32; m >= 1 && n > 1; m >>= 1, n >>= 1)
    if (lane & m) row += n / 2;
  return row;
}

template <int N, int M>
struct RowHalver {
  TFA_DEV static void run(float* v, int lane) {
    const bool upper = (lane & M) != 0;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const float keep = upper ? v[j + N / 2] : v[j];
      const float send = upper ? v[j] : v[j + N / 2];
      v[j] = keep + __shfl_xor(send, M, kWave);
    }
    RowHalver<N / 2, M / 2>::run(v, lane);
  }
};
template <int M>
struct RowHalver<1, M> {
  TFA_DEV static void run(float* v, int lane) {
#pragma unroll
    for (int m = M; m >= 1; m >>= 1) v[0] += __shfl_xor(v[0], m, kWave);
  }
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
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
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
// Sum of the first `ks` (<= MAXKS) of p[0], p[stride], p[2 stride], ... in split
// order, with every load issued before the first add: one memory round trip,
// not one per split (a runtime-bounded loop waits for each load in turn).
constexpr int kMaxSplitsK = 8;
template <int MAXKS = kMaxSplitsK>
TFA_DEV float sum_splits(const float* p, size_t stride, int ks) {
  float v[MAXKS];
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) v[s] = s < ks ? p[s * stride] : 0.f;
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < MAXKS; ++s)
    if (s < ks) acc += v[s];
  return acc;
}

// The same for eight consecutive floats (two 16-byte loads per split);
// p 16-byte aligned, stride a multiple of 4.
template <int MAXKS = kMaxSplitsK>
TFA_DEV void sum_splits8(const float* p, size_t stride, int ks, float* acc) {
  float4 v[MAXKS][2];
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) {
    if (s < ks) {
      const float4* q = reinterpret_cast<const float4*>(p + s * stride);
      v[s][0] = q[0];
      v[s][1] = q[1];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
  for (int s = 0; s < MAXKS; ++s) {
    if (s < ks) {
      acc[0] += v[s][0].x; acc[1] += v[s][0].y; acc[2] += v[s][0].z; acc[3] += v[s][0].w;
      acc[4] += v[s][1].x; acc[5] += v[s][1].y; acc[6] += v[s][1].z; acc[7] += v[s][1].w;
    }
  }
}

// 1/sqrt(x) with correctly rounded sqrt and division: the value torch's CPU
// `rsqrt` returns for the same f32 input.
TFA_DEV float rsqrt_rn(float x) { return 1.0f / __fsqrt_rn(x); }

TFA_DEV float silu(float x) { return x / (1.0f + __expf(-x)); }

// --------------------------------------------------- last block finishes
// A group of blocks each publishes a slice of a result, then one of them --
// whichever arrives last -- runs the step that needs the whole result. The
// counter resets itself, so the same buffer serves every launch (and every
// replay of a captured graph) without a memset.
//
// Coherence without whole-cache maintenance: on gfx950 each XCD has its own
// L2, and an agent-scope fence (`__threadfence`) writes back and invalidates
// that entire L2 -- once per block, serialised, it costs milliseconds over a
// 10k-block grid. So slices are published with agent-scope atomic stores
// (`global_store ... sc1`, written through to the coherent level) and read
// back with agent-scope atomic loads (`global_load ... sc1`). Each thread waits
// for its own publishing stores to complete (`s_waitcnt`) before the block
// barrier, and only then does one thread bump the counter: every slice a block
// published is visible at agent scope before its arrival is counted. Data that
// is only consumed by a later kernel uses ordinary stores (the kernel boundary
// orders it).
TFA_DEV void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TFA_DEV void publish(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TFA_DEV float fetch(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TFA_DEV int fetch(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true in exactly one block of the group. Every thread of the block
// must call it (it synchronises the block). Slices must have been written with
// publish() and must be read with fetch().
TFA_DEV bool arrive_last(unsigned int* counter, unsigned int group_size, int* flag_smem) {
  __builtin_amdgcn_s_waitcnt(0);    // this thread's published stores are complete
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int prev =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = (prev == group_size - 1);
    // No other block of this launch touches the counter after the last arrival.
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag_smem = last;
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return *flag_smem != 0;
}

}  // namespace tfa
