// RMSNorm family: plain rows, fused residual-add + norm over rows, and the
// single-row "reduce split-K partials, add residual, norm" form.
//
// Rounding points (each value lands in bf16 exactly where the reference's
// torch spelling lands it):
//   MODE 0 (Qwen3 / MiniCPM3, reference examples/qwen3_1_7b-tilelang/fast/kernels.py:58-79):
//            y = bf16( bf16(x * r) * gamma ),  r = 1/sqrt(mean(x^2) + eps)
//   MODE 1 (Qwen3.5 prefill, examples/qwen3_8_27b_prefill-tilelang/kernels/elementwise.py:21-68):
//            y = bf16( (x * r) * (1 + gamma) ) in f32
//   MODE 2 (MiniCPM3 final norm + the head's divide, examples/minicpm3_4b-cutedsl/model.py
//           final_rms_norm and lm_head):
//            y = bf16( bf16( bf16(x * r) * gamma ) / d ), a correctly rounded divide
// The fused add lands the sum in bf16 first (r' = bf16(x + res)) and normalises
// that landed value, which is what `Hout = A + ...; Xn = norm(Hout)` does in
// examples/qwen3_1_7b-tilelang/fast/kernels.py:82-116.
#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

template <int MODE>
TFA_DEV float norm_scale(float x, float r, float g, float d) {
  if (MODE == 0) return round_bf(round_bf(x * r) * g);
  if (MODE == 2) return round_bf(__fdiv_rn(round_bf(round_bf(x * r) * g), d));
  return (x * r) * (g + 1.0f);
}

// norm_scale for the two bf16 values of a packed word, landed as a packed
// word: every landing converts both values in one v_cvt_pk_bf16_f32 (the same
// round-to-nearest-even), and the final landing is the stored word itself.
template <int MODE>
TFA_DEV uint32_t norm_pair(uint32_t hw, float r, uint32_t gw, float d) {
  const float h0 = lo_bf(hw), h1 = hi_bf(hw), g0 = lo_bf(gw), g1 = hi_bf(gw);
  if (MODE == 1) return pack_bf((h0 * r) * (g0 + 1.0f), (h1 * r) * (g1 + 1.0f));
  const uint32_t t = pack_bf(h0 * r, h1 * r);   // bf16(x * r)
  const uint32_t u = pack_bf(lo_bf(t) * g0, hi_bf(t) * g1);
  if (MODE == 0) return u;
  return pack_bf(__fdiv_rn(lo_bf(u), d), __fdiv_rn(hi_bf(u), d));
}

// One wave per row; each lane owns NC 16-byte vectors of the row, so the whole
// row sits in registers between the sum of squares and the write. NT: the
// outputs go out with non-temporal stores (many-row calls, where nothing reads
// them back from L2 right away): [4096, 2048] add + norm 12.4 -> 11.35 us.
// (Issuing the norm scale's loads with the row's, before the reduction, was
// measured slower: 11.8-12.8 us.)
template <int NC, bool ADD, int MODE, bool NT>
__global__ __launch_bounds__(256) void rms_rows_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ y,
    uint16_t* __restrict__ res_out, int rows, int H, float eps, float div) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const int nvec = H >> 3;
  const size_t base = static_cast<size_t>(row) * H;

  uint4 xv[NC];
  uint4 rv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int v = lane + c * kWave;
    if (v < nvec) {
      xv[c] = ld16_stream(x + base + 8 * v);
      if (ADD) rv[c] = ld16_stream(res + base + 8 * v);
    }
  }
  // the add lands each pair of sums in bf16 with one convert (that packed word
  // is also the residual output); squares summed in element order
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int v = lane + c * kWave;
    if (v < nvec) {
      uint32_t w[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
      if (ADD) {
        const uint32_t q[4] = {rv[c].x, rv[c].y, rv[c].z, rv[c].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = pack_bf(lo_bf(w[k]) + lo_bf(q[k]), hi_bf(w[k]) + hi_bf(q[k]));
        xv[c] = make_uint4(w[0], w[1], w[2], w[3]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float h0 = lo_bf(w[k]), h1 = hi_bf(w[k]);
        ss += h0 * h0;
        ss += h1 * h1;
      }
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrt_rn(ss / static_cast<float>(H) + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int v = lane + c * kWave;
    if (v < nvec) {
      const uint4 gv = ld16(gamma + 8 * v);
      const uint4 yv = make_uint4(norm_pair<MODE>(xv[c].x, r, gv.x, div), norm_pair<MODE>(xv[c].y, r, gv.y, div),
                                  norm_pair<MODE>(xv[c].z, r, gv.z, div), norm_pair<MODE>(xv[c].w, r, gv.w, div));
      if (NT) {
        st16_stream(y + base + 8 * v, yv);
        if (ADD) st16_stream(res_out + base + 8 * v, xv[c]);
      } else {
        st16(y + base + 8 * v, yv);
        if (ADD) st16(res_out + base + 8 * v, xv[c]);
      }
    }
  }
}

// Row count from which the outputs are streamed (non-temporal) rather than
// left in L2 for a consumer: a decode step's few rows stay cached.
constexpr int kStreamRows = 256;

template <int NC>
int launch_rows(const void* x, const void* res, const void* gamma, void* y, void* res_out,
                int rows, int H, float eps, int mode, float div, hipStream_t s) {
  const dim3 block(256);
  const dim3 grid((rows + 3) / 4);
  auto X = static_cast<const uint16_t*>(x);
  auto R = static_cast<const uint16_t*>(res);
  auto G = static_cast<const uint16_t*>(gamma);
  auto Y = static_cast<uint16_t*>(y);
  auto RO = static_cast<uint16_t*>(res_out);
  if (rows >= kStreamRows) {
    if (res) {
      if (mode == 0) rms_rows_kernel<NC, true, 0, true><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
      else rms_rows_kernel<NC, true, 1, true><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
    } else {
      if (mode == 0) rms_rows_kernel<NC, false, 0, true><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
      else if (mode == 1) rms_rows_kernel<NC, false, 1, true><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
      else rms_rows_kernel<NC, false, 2, true><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
    }
    return launched("rms_norm_rows");
  }
  if (res) {
    if (mode == 0) rms_rows_kernel<NC, true, 0, false><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
    else rms_rows_kernel<NC, true, 1, false><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
  } else {
    if (mode == 0) rms_rows_kernel<NC, false, 0, false><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
    else if (mode == 1) rms_rows_kernel<NC, false, 1, false><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
    else rms_rows_kernel<NC, false, 2, false><<<grid, block, 0, s>>>(X, R, G, Y, RO, rows, H, eps, div);
  }
  return launched("rms_norm_rows");
}

int dispatch_rows(const void* x, const void* res, const void* gamma, void* y, void* res_out,
                  int64_t rows, int64_t H, float eps, int mode, hipStream_t s, float div = 1.f) {
  const int nc = static_cast<int>((H / 8 + kWave - 1) / kWave);
  switch (nc) {
#define TFA_NC(n) case n: return launch_rows<n>(x, res, gamma, y, res_out, (int)rows, (int)H, eps, mode, div, s);
    TFA_NC(1) TFA_NC(2) TFA_NC(3) TFA_NC(4) TFA_NC(5) TFA_NC(6) TFA_NC(7) TFA_NC(8)
    TFA_NC(9) TFA_NC(10) TFA_NC(11) TFA_NC(12) TFA_NC(13) TFA_NC(14) TFA_NC(15) TFA_NC(16)
#undef TFA_NC
    default: return fail(TFA_ERR_SHAPE, "rms_norm: hidden %lld exceeds 8192", (long long)H);
  }
}

int check_rows(const void* x, const void* gamma, const void* y, int64_t rows, int64_t H, int mode,
               const char* fn) {
  if (rows < 0 || rows > (1LL << 31) - 1) return fail(TFA_ERR_SHAPE, "%s: rows %lld out of range", fn, (long long)rows);
  if (H <= 0 || H % 8 != 0 || H > 8192) return fail(TFA_ERR_SHAPE, "%s: hidden %lld must be a positive multiple of 8, at most 8192", fn, (long long)H);
  if (mode != 0 && mode != 1) return fail(TFA_ERR_ARG, "%s: mode %d is not 0 or 1", fn, mode);
  if (rows == 0) return TFA_OK;  // nothing to touch; empty tensors may be null
  if (!x || !gamma || !y) return fail(TFA_ERR_NULL, "%s: null pointer", fn);
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(y)) return fail(TFA_ERR_ALIGN, "%s: tensors must be 16-byte aligned", fn);
  return TFA_OK;
}

// Single row: Hout = A + bf16(sum_s P[s]); Xn = norm(Hout) * gamma (MODE 0).
// One block; the row is staged in LDS between the sum of squares and the write.
__global__ __launch_bounds__(256) void resid_rms_partials_kernel(
    const uint16_t* __restrict__ a, const float* __restrict__ p, int sk,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ hout,
    uint16_t* __restrict__ xn, int H, float eps) {
  extern __shared__ float row[];
  __shared__ float red[16];
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    float acc = 0.f;
#pragma unroll 8
    for (int s = 0; s < sk; ++s) acc += p[static_cast<size_t>(s) * H + i];
    const float v = round_bf(bf2f(a[i]) + round_bf(acc));
    hout[i] = static_cast<uint16_t>(f2bf(v));
    row[i] = v;
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float r = rsqrt_rn(ss / static_cast<float>(H) + eps);
  for (int i = threadIdx.x; i < H; i += blockDim.x)
    xn[i] = static_cast<uint16_t>(f2bf(round_bf(round_bf(row[i] * r) * bf2f(gamma[i]))));
}

}  // namespace

extern "C" {

int tfa_rms_norm(const void* x, const void* gamma, void* y, int64_t rows, int64_t hidden,
                 float eps, int mode, hipStream_t stream) {
  int st = check_rows(x, gamma, y, rows, hidden, mode, "tfa_rms_norm");
  if (st != TFA_OK) return st;
  if (rows == 0) return TFA_OK;
  return dispatch_rows(x, nullptr, gamma, y, nullptr, rows, hidden, eps, mode, stream);
}

int tfa_rms_norm_div(const void* x, const void* gamma, void* y, int64_t rows, int64_t hidden, float eps,
                     float divisor, hipStream_t stream) {
  int st = check_rows(x, gamma, y, rows, hidden, 0, "tfa_rms_norm_div");
  if (st != TFA_OK) return st;
  TFA_REQUIRE(divisor != 0.f && divisor == divisor, TFA_ERR_ARG, "tfa_rms_norm_div: divisor must be nonzero");
  if (rows == 0) return TFA_OK;
  return dispatch_rows(x, nullptr, gamma, y, nullptr, rows, hidden, eps, 2, stream, divisor);
}

int tfa_add_rms_norm(const void* x, const void* residual, const void* gamma, void* y,
                     void* residual_out, int64_t rows, int64_t hidden, float eps, int mode,
                     hipStream_t stream) {
  int st = check_rows(x, gamma, y, rows, hidden, mode, "tfa_add_rms_norm");
  if (st != TFA_OK || rows == 0) return st;
  TFA_NONNULL(residual);
  TFA_NONNULL(residual_out);
  TFA_ALIGN16(residual);
  TFA_ALIGN16(residual_out);
  if (rows == 0) return TFA_OK;
  return dispatch_rows(x, residual, gamma, y, residual_out, rows, hidden, eps, mode, stream);
}

int tfa_resid_rms_norm_partials(const void* a, const float* partials, int64_t splits,
                                const void* gamma, void* h_out, void* xn, int64_t hidden,
                                float eps, hipStream_t stream) {
  TFA_NONNULL(a);
  TFA_NONNULL(partials);
  TFA_NONNULL(gamma);
  TFA_NONNULL(h_out);
  TFA_NONNULL(xn);
  TFA_REQUIRE(hidden > 0 && hidden <= 8192, TFA_ERR_SHAPE, "tfa_resid_rms_norm_partials: hidden %lld not in [1, 8192]", (long long)hidden);
  TFA_REQUIRE(splits > 0 && splits <= 4096, TFA_ERR_SHAPE, "tfa_resid_rms_norm_partials: splits %lld not in [1, 4096]", (long long)splits);
  resid_rms_partials_kernel<<<1, 256, hidden * sizeof(float), stream>>>(
      static_cast<const uint16_t*>(a), partials, (int)splits, static_cast<const uint16_t*>(gamma),
      static_cast<uint16_t*>(h_out), static_cast<uint16_t*>(xn), (int)hidden, eps);
  return launched("resid_rms_norm_partials");
}

}  // extern "C"
