// Dense bf16 GEMM for the prefill projections: C[M, N] = A[M, K] . B[N, K]^T
// (activations and weights both K-contiguous, f32 accumulate) on
// v_mfma_f32_32x32x16_bf16, with fused epilogues:
//
//   store         C = bf16(acc)
//   residual      C = bf16(R + bf16(acc))                      (o_proj + residual)
//   qk_norm_rope  (a separate in-place pass over the qkv projection output,
//                 laid out per token [q_0 | gate_0 | ... | q_{H-1} | gate_{H-1} |
//                 k_0 .. k_{G-1} | v_0 .. v_{G-1}], 256 per slice): q and k slices
//                 get the per-head RMSNorm with (1 + gamma) in f32 and rotate-half
//                 RoPE on their leading 64 dims (bf16 products and sum); gate and
//                 v slices are left as the projection landed them.
//
// The products themselves are plain GEMMs and run on hipBLASLt (bf16 in, f32
// compute, bf16 out, no workspace), one cached plan per device and shape:
// measured 1.2-1.4 PFLOP/s on these shapes against 0.6-0.9 for the kernel below.
// The residual epilogue is then a separate element-wise pass with the
// reference's rounding, and qk_norm_rope runs in place as before.
//
// gemm_nt_kernel, the native MFMA GEMM, serves shapes hipBLASLt returns no plan
// for, and every shape when TFA_GEMM_NATIVE=1 is set in the environment (read
// once). Block tile 256 x 256 x 64, four waves of 128 x 128 (16 accumulator
// tiles of 32 x 32). A and B stages stream global -> LDS with
// global_load_lds_dwordx4, double-buffered; rows of 8 16-byte chunks are
// stored at chunk ^ ((row >> 1) & 7) so the 16-row operand reads are
// conflict-free.
//
// Reference (jingchangshi/TileFoundry): examples/qwen3_8_27b_prefill-tilelang/kernels/gemm.py:104-356
// (gemm_kernel, "qk_norm_rope" epilogue :226-300, "residual" :193-198), model.py:271-303,326-333.
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

TFA_DEV bf16x8 as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_F32 = 2 };

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
  const uint16_t* cos_t;  // [M, rot] rows = positions
  const uint16_t* sin_t;
  int rot, q_tiles, k_tiles;
  float eps;
};

TFA_DEV int swz(int row) { return (row >> 1) & 7; }

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) with expcnt / lgkmcnt left open.
constexpr int kWaitVm16 = waitcnt_vm(16);
constexpr int kWaitVm0 = waitcnt_vm(0);

template <int EPI>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(const GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t smem[2][kBM + kBN][kBK];   // per stage: A rows, then B rows

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int n32 = lane & 31;
  const int kg = lane >> 5;
  const int wm = (wid >> 1) * 128, wn = (wid & 1) * 128;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

  // stage loads: instruction j covers LDS rows 8j .. 8j+7 of the stage (A rows
  // 0..255, B rows 256..511); lane l lands at row 8j + l/8, chunk slot l % 8 and
  // so loads logical chunk (l % 8) ^ swz(row). Wave w issues j = 16w .. 16w+15.
  auto load_stage = [&](int kt, int buf) __attribute__((always_inline)) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = 16 * wid + i;                 // wave-uniform
      const int row = 8 * j + (lane >> 3);        // stage row
      const int q = (lane & 7) ^ swz(row);
      const uint16_t* src = row < kBM ? a.a + static_cast<size_t>(min(m0 + row, a.M - 1)) * a.lda
                                      : a.b + static_cast<size_t>(n0 + row - kBM) * a.ldb;
      lds_dma16(src + k0 + 8 * q, lds_offset(&smem[buf][8 * j][0]));
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int nk = a.K / kBK;
  const int sx = swz(n32);   // the swizzle of every operand row this lane reads
  load_stage(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) {
      load_stage(kt + 1, buf ^ 1);
      __builtin_amdgcn_s_waitcnt(kWaitVm16);   // stage kt landed; stage kt + 1 stays in flight
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
    }
    block_barrier();   // every wave's stage kt landed
    const uint16_t* arow = &smem[buf][wm + n32][0];
    const uint16_t* brow = &smem[buf][kBM + wn + n32][0];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int off = 8 * ((2 * ks + kg) ^ sx);
      uint4 aop[4], bop[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        aop[i] = *reinterpret_cast<const uint4*>(arow + 32 * i * kBK + off);
        bop[i] = *reinterpret_cast<const uint4*>(brow + 32 * i * kBK + off);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf8(aop[i]), as_bf8(bop[j]), acc[i][j], 0, 0, 0);
    }
    block_barrier();   // every wave is done with buf before it is refilled
  }

  // acc[i][j][4t + r]: row m0 + wm + 32i + 8t + 4kg + r, column n0 + wn + 32j + n32
  {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t row = m0 + wm + 32 * i + 8 * t + 4 * kg + r;
          if (row >= static_cast<size_t>(a.M)) continue;   // rows past M read row M - 1
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int col = n0 + wn + 32 * j + n32;
            if (EPI == EPI_F32) {
              a.cf[row * a.ldc + col] = acc[i][j][4 * t + r];
              continue;
            }
            float v = round_bf(acc[i][j][4 * t + r]);
            if (EPI == EPI_RESID) v = round_bf(bf2f(a.res[row * a.ldr + col]) + v);
            a.c[row * a.ldc + col] = static_cast<uint16_t>(f2bf(v));
          }
        }
    return;
  }

}

// In place on the packed qkv projection output [n, ldc]: one wave per (token,
// q or k head slice of 256): x -> bf16(x * rsqrt(mean x^2 + eps) * (1 + gamma))
// in f32, then rotate-half RoPE on dims 0..63 with each product and the sum
// landing in bf16 (partners 32 apart: lane l and l ^ 8 hold them). Lane l owns
// dims 4l .. 4l+3.
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(
    uint16_t* __restrict__ qkv, int ldc, int n, int heads, int kv_heads, const uint16_t* __restrict__ gq,
    const uint16_t* __restrict__ gk, const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t,
    float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int slices = heads + kv_heads;
  const int wv = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  if (wv >= n * slices) return;
  const int row = wv / slices, sl = wv % slices;
  const bool is_q = sl < heads;
  uint16_t* p = qkv + static_cast<size_t>(row) * ldc + (is_q ? sl * 512 : heads * 512 + (sl - heads) * 256) + 4 * lane;
  const uint16_t* gamma = (is_q ? gq : gk) + 4 * lane;
  const uint2 xv = *reinterpret_cast<const uint2*>(p);
  const uint2 gv = *reinterpret_cast<const uint2*>(gamma);
  float x[4] = {lo_bf(xv.x), hi_bf(xv.x), lo_bf(xv.y), hi_bf(xv.y)};
  const float g[4] = {lo_bf(gv.x), hi_bf(gv.x), lo_bf(gv.y), hi_bf(gv.y)};
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss = fmaf(x[i], x[i], ss);
  const float inv = rsqrt_rn(wave_sum(ss) / 256.0f + eps);
  float y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i] = round_bf(x[i] * inv * (1.0f + g[i]));
  float partner[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) partner[i] = __shfl_xor(y[i], 8, kWave);
  if (lane < 16) {   // dims 0..63
    const uint2 cv = *reinterpret_cast<const uint2*>(cos_t + static_cast<size_t>(row) * 64 + 4 * lane);
    const uint2 sv = *reinterpret_cast<const uint2*>(sin_t + static_cast<size_t>(row) * 64 + 4 * lane);
    const float c[4] = {lo_bf(cv.x), hi_bf(cv.x), lo_bf(cv.y), hi_bf(cv.y)};
    const float s4[4] = {lo_bf(sv.x), hi_bf(sv.x), lo_bf(sv.y), hi_bf(sv.y)};
    const float sign = lane < 8 ? -1.0f : 1.0f;   // rotate_half: first half pairs with -x[d + 32]
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = round_bf(round_bf(y[i] * c[i]) + round_bf(sign * partner[i] * s4[i]));
  }
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf(y[0], y[1]), pack_bf(y[2], y[3]));
}

template <int EPI>
int launch(const GemmArgs& g, hipStream_t st, const char* name) {
  const dim3 grid((unsigned)(g.N / kBN), (unsigned)((g.M + kBM - 1) / kBM));
  gemm_nt_kernel<EPI><<<grid, kThreads, 0, st>>>(g);
  return launched(name);
}

int check_gemm(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
               int64_t ldc, const char* fn) {
  if (!a || !b || !c) return fail(TFA_ERR_NULL, "%s: null pointer argument", fn);
  if (m < 1 || n < kBN || n % kBN || k < kBK || k % kBK || m > (1 << 24) || n > (1 << 24))
    return fail(TFA_ERR_SHAPE, "%s: m %lld must be positive, n %lld a multiple of 256, k %lld of 64", fn,
                (long long)m, (long long)n, (long long)k);
  if (lda < k || ldb < k || ldc < n || lda % 8 || ldb % 8)
    return fail(TFA_ERR_SHAPE, "%s: leading dimensions too small or not multiples of 8", fn);
  if (!aligned16(a) || !aligned16(b)) return fail(TFA_ERR_ALIGN, "%s: a / b not 16-byte aligned", fn);
  return TFA_OK;
}

GemmArgs make(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
              int64_t ldc) {
  GemmArgs g{};
  g.a = static_cast<const uint16_t*>(a);
  g.b = static_cast<const uint16_t*>(b);
  g.c = static_cast<uint16_t*>(c);
  g.M = (int)m; g.N = (int)n; g.K = (int)k;
  g.lda = (int)lda; g.ldb = (int)ldb; g.ldc = (int)ldc;
  return g;
}

// c[r, j] = bf16(res[r, j] + c[r, j]) over [m, n]: the o_proj residual after
// the library product landed bf16(A . B^T) in c. 8 elements per thread.
__global__ __launch_bounds__(kThreads) void residual_add_kernel(uint16_t* c, int ldc, const uint16_t* res, int ldr,
                                                                 int m, int n) {
  const int per_row = n / 8;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (e >= static_cast<int64_t>(m) * per_row) return;
  const int r = static_cast<int>(e / per_row), j = static_cast<int>(e % per_row) * 8;
  uint16_t* cp = c + static_cast<size_t>(r) * ldc + j;
  float x[8], y[8];
  unpack8(ld16(cp), x);
  unpack8(ld16(res + static_cast<size_t>(r) * ldr + j), y);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = round_bf(y[i] + x[i]);
  st16(cp, pack8(x));
}

// hipBLASLt plan for row-major C[m, n] = A[m, k] . B[n, k]^T: in column-major
// terms C^T (n x m, ld ldc) = op_T(B^T stored k x n, ld ldb) . (A^T stored k x m,
// ld lda).
struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

std::mutex g_lt_mu;
std::map<int, hipblasLtHandle_t> g_lt_handles;
std::map<std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, bool>, LtPlan> g_lt_plans;

bool force_native() {
  static const bool f = [] {
    const char* v = std::getenv("TFA_GEMM_NATIVE");
    return v && v[0] == '1';
  }();
  return f;
}

// The plan for this device, shape and output type (created once; ok == false
// when the library has none, and the caller uses the native kernel).
const LtPlan* lt_plan(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, bool out_f32,
                      hipblasLtHandle_t* handle) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_lt_mu);
  auto hit = g_lt_handles.find(dev);
  if (hit == g_lt_handles.end()) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return nullptr;
    hit = g_lt_handles.emplace(dev, h).first;
  }
  *handle = hit->second;
  const auto key = std::make_tuple(dev, m, n, k, lda, ldb, ldc, out_f32);
  auto it = g_lt_plans.find(key);
  if (it != g_lt_plans.end()) return &it->second;
  LtPlan p;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulPreference_t pref = nullptr;
  const uint64_t ws = 0;
  int found = 0;
  constexpr int kCandidates = 16;   // the first answer can still ask for workspace
  hipblasLtMatmulHeuristicResult_t res[kCandidates]{};
  p.ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_16BF, k, n, ldb) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, k, m, lda) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatrixLayoutCreate(&p.lc, out_f32 ? HIP_R_32F : HIP_R_16BF, n, m, ldc) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) ==
             HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulAlgoGetHeuristic(*handle, p.desc, p.lw, p.la, p.lc, p.lc, pref, kCandidates, res, &found) ==
             HIPBLAS_STATUS_SUCCESS;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  bool picked = false;
  for (int i = 0; p.ok && i < found && !picked; ++i) {
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) {
      p.algo = res[i].algo;
      picked = true;
    }
  }
  p.ok = p.ok && picked;
  return &g_lt_plans.emplace(key, p).first->second;
}

// C = bf16(A . B^T) (or the f32 A . B^T) through the library; false when there
// is no plan (the caller then launches the native kernel), or with *status set
// on a failed call.
bool lt_gemm(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
             int64_t ldc, hipStream_t st, int* status, bool out_f32 = false) {
  *status = TFA_OK;
  if (force_native()) return false;
  hipblasLtHandle_t h = nullptr;
  const LtPlan* p = lt_plan(m, n, k, lda, ldb, ldc, out_f32, &h);
  if (!p || !p->ok) return false;
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t r = hipblasLtMatmul(h, p->desc, &alpha, b, p->lw, a, p->la, &beta, c, p->lc, c, p->lc,
                                            &p->algo, nullptr, 0, st);
  if (r != HIPBLAS_STATUS_SUCCESS) *status = fail(TFA_ERR_LAUNCH, "hipblasLtMatmul failed with status %d", (int)r);
  return true;
}

}  // namespace

extern "C" {

int tfa_gemm_nt(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb,
                int64_t ldc, const void* residual, int64_t ldr, hipStream_t stream) {
  int st = check_gemm(a, b, c, m, n, k, lda, ldb, ldc, "tfa_gemm_nt");
  if (st != TFA_OK) return st;
  GemmArgs g = make(a, b, c, m, n, k, lda, ldb, ldc);
  if (residual) {
    TFA_REQUIRE(ldr >= n, TFA_ERR_SHAPE, "tfa_gemm_nt: ldr %lld < n %lld", (long long)ldr, (long long)n);
    TFA_REQUIRE(ldr % 8 == 0 && ldc % 8 == 0 && aligned16(residual) && aligned16(c), TFA_ERR_ALIGN,
                "tfa_gemm_nt: residual / c rows must be 16-byte aligned");
  }
  if (lt_gemm(a, b, c, m, n, k, lda, ldb, ldc, stream, &st)) {
    if (st != TFA_OK || !residual) return st;
    const int64_t threads = m * (n / 8);
    residual_add_kernel<<<(unsigned)((threads + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
        static_cast<uint16_t*>(c), (int)ldc, static_cast<const uint16_t*>(residual), (int)ldr, (int)m, (int)n);
    return launched("gemm_nt_residual_add");
  }
  if (residual) {
    g.res = static_cast<const uint16_t*>(residual);
    g.ldr = (int)ldr;
    return launch<EPI_RESID>(g, stream, "gemm_nt_residual");
  }
  return launch<EPI_STORE>(g, stream, "gemm_nt");
}

int tfa_gemm_nt_f32(const void* a, const void* b, float* c, int64_t m, int64_t n, int64_t k, int64_t lda,
                    int64_t ldb, int64_t ldc, hipStream_t stream) {
  int st = check_gemm(a, b, c, m, n, k, lda, ldb, ldc, "tfa_gemm_nt_f32");
  if (st != TFA_OK) return st;
  if (lt_gemm(a, b, c, m, n, k, lda, ldb, ldc, stream, &st, true)) return st;
  GemmArgs g = make(a, b, nullptr, m, n, k, lda, ldb, ldc);
  g.cf = c;
  return launch<EPI_F32>(g, stream, "gemm_nt_f32");
}

int tfa_qkv_norm_rope(const void* hn, const void* w_qkv, void* out, int64_t n, int64_t hidden, int64_t heads,
                      int64_t kv_heads, int64_t head_dim, const void* gamma_q, const void* gamma_k, float eps,
                      const void* cos_t, const void* sin_t, int64_t rot, hipStream_t stream) {
  TFA_REQUIRE(head_dim == 256, TFA_ERR_SHAPE, "tfa_qkv_norm_rope: head_dim %lld, only 256 supported", (long long)head_dim);
  TFA_REQUIRE(rot == 64, TFA_ERR_SHAPE, "tfa_qkv_norm_rope: rot %lld, only 64 supported", (long long)rot);
  TFA_REQUIRE(heads >= 1 && kv_heads >= 1, TFA_ERR_SHAPE, "tfa_qkv_norm_rope: empty head counts");
  TFA_NONNULL(gamma_q);
  TFA_NONNULL(gamma_k);
  TFA_NONNULL(cos_t);
  TFA_NONNULL(sin_t);
  const int64_t width = (2 * heads + 2 * kv_heads) * head_dim;
  int st = check_gemm(hn, w_qkv, out, n, width, hidden, hidden, hidden, width, "tfa_qkv_norm_rope");
  if (st != TFA_OK) return st;
  if (!lt_gemm(hn, w_qkv, out, n, width, hidden, hidden, hidden, width, stream, &st)) {
    GemmArgs g = make(hn, w_qkv, out, n, width, hidden, hidden, hidden, width);
    st = launch<EPI_STORE>(g, stream, "qkv_gemm");
  }
  if (st != TFA_OK) return st;
  const int64_t waves = n * (heads + kv_heads);
  qk_norm_rope_kernel<<<(unsigned)((waves + 3) / 4), kThreads, 0, stream>>>(
      static_cast<uint16_t*>(out), (int)width, (int)n, (int)heads, (int)kv_heads,
      static_cast<const uint16_t*>(gamma_q), static_cast<const uint16_t*>(gamma_k),
      static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t), eps);
  return launched("qk_norm_rope");
}

}  // extern "C"
