// Measurement utilities.
// * copy_stream: a device-to-device copy built from the same 16-byte
//   non-temporal loads and plain 16-byte stores the decode kernels use. It gives
//   the HBM bandwidth this device actually sustains for that access pattern, and
//   it is the calibration dispatch for the FETCH_SIZE / WRITE_SIZE counters (a
//   copy of known size read through the same load path as the kernels measured).
// * read_rows: the decode GEMV's weight stream alone -- one-shot 256-thread
//   blocks of R rows, each wave a contiguous quarter of every row in 16-byte
//   non-temporal loads, all issued before any is read -- with no arithmetic
//   beyond folding the loaded words into one value per block. Its time per
//   launch is the floor of that access pattern for a given matrix.
#include "abi_util.h"
#include "common.h"

using namespace tfa;

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 16;  // 16-byte vectors per thread per block tile

// Block b copies the contiguous tile [b * 64 KiB, (b + 1) * 64 KiB) (the last
// tile may be short); every load of the tile is issued before any store.
__global__ __launch_bounds__(kThreads) void copy_stream_kernel(const uint4* __restrict__ src,
                                                               uint4* __restrict__ dst,
                                                               size_t n16) {
  const size_t base = static_cast<size_t>(blockIdx.x) * kThreads * kChunk;
  uint4 v[kChunk];
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    const size_t i = base + static_cast<size_t>(u) * kThreads + threadIdx.x;
    v[u] = i < n16 ? ld16_stream(src + i) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int u = 0; u < kChunk; ++u) {
    const size_t i = base + static_cast<size_t>(u) * kThreads + threadIdx.x;
    if (i < n16) dst[i] = v[u];
  }
}

template <int R, int NCH>
__global__ __launch_bounds__(kThreads) void read_rows_kernel(const uint16_t* __restrict__ w, int rows, int k,
                                                             float* __restrict__ out) {
  __shared__ float red[kThreads / kWave];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int kq = k / 4, nch = kq / 8;
  const int row0 = blockIdx.x * R;
  uint4 v[R][NCH];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      v[r][j] = ld16_stream(w + static_cast<size_t>(min(row0 + r, rows - 1)) * k + wid * kq +
                            8 * min(lane + j * kWave, nch - 1));
  uint32_t x = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < NCH; ++j) x ^= v[r][j].x ^ v[r][j].y ^ v[r][j].z ^ v[r][j].w;
  const float s = wave_sum(__uint_as_float(x & 0x3FFFFFFFu));
  if (lane == 0) red[wid] = s;
  lds_barrier();
  if (threadIdx.x == 0) out[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

template <int R>
void launch_read_rows(const uint16_t* w, int rows, int k, float* out, hipStream_t st) {
  const unsigned blocks = static_cast<unsigned>((rows + R - 1) / R);
  switch ((k / 4 / 8 + kWave - 1) / kWave) {
    case 1: read_rows_kernel<R, 1><<<blocks, kThreads, 0, st>>>(w, rows, k, out); break;
    case 2: read_rows_kernel<R, 2><<<blocks, kThreads, 0, st>>>(w, rows, k, out); break;
    case 3: read_rows_kernel<R, 3><<<blocks, kThreads, 0, st>>>(w, rows, k, out); break;
    default: read_rows_kernel<R, 4><<<blocks, kThreads, 0, st>>>(w, rows, k, out); break;
  }
}

}  // namespace

extern "C" int tfa_read_rows(const void* w, int64_t rows, int64_t k, int64_t rows_per_block, float* out,
                             hipStream_t stream) {
  TFA_NONNULL(w);
  TFA_NONNULL(out);
  TFA_REQUIRE(rows >= 1 && rows <= (1 << 24) && k >= 32 && k % 32 == 0 && k <= 8192, TFA_ERR_SHAPE,
              "tfa_read_rows: rows %lld, k %lld (a multiple of 32, at most 8192)", (long long)rows, (long long)k);
  TFA_ALIGN16(w);
  const auto W = static_cast<const uint16_t*>(w);
  switch (rows_per_block) {
    case 2: launch_read_rows<2>(W, (int)rows, (int)k, out, stream); break;
    case 4: launch_read_rows<4>(W, (int)rows, (int)k, out, stream); break;
    case 6: launch_read_rows<6>(W, (int)rows, (int)k, out, stream); break;
    case 8: launch_read_rows<8>(W, (int)rows, (int)k, out, stream); break;
    default: return fail(TFA_ERR_SHAPE, "tfa_read_rows: rows_per_block %lld not in {2, 4, 6, 8}", (long long)rows_per_block);
  }
  return launched("read_rows");
}

extern "C" int tfa_copy_stream(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
  TFA_NONNULL(src);
  TFA_NONNULL(dst);
  TFA_REQUIRE(bytes >= 0 && bytes % 16 == 0, TFA_ERR_SHAPE, "tfa_copy_stream: %lld bytes is not a multiple of 16", (long long)bytes);
  TFA_ALIGN16(src);
  TFA_ALIGN16(dst);
  if (bytes == 0) return TFA_OK;
  const size_t n16 = static_cast<size_t>(bytes) / 16;
  const size_t per_block = static_cast<size_t>(kThreads) * kChunk;
  const unsigned blocks = static_cast<unsigned>((n16 + per_block - 1) / per_block);
  copy_stream_kernel<<<blocks, kThreads, 0, stream>>>(static_cast<const uint4*>(src),
                                                      static_cast<uint4*>(dst), n16);
  return launched("copy_stream");
}
