// Measurement utility: a device-to-device copy built from the same 16-byte
// non-temporal loads and plain 16-byte stores the decode kernels use. It gives
// the HBM bandwidth this device actually sustains for that access pattern, and
// it is the calibration dispatch for the FETCH_SIZE / WRITE_SIZE counters (a
// copy of known size read through the same load path as the kernels measured).
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

}  // namespace

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
