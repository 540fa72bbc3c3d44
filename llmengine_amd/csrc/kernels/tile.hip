// Raw Q8_0 [N, K] -> Q8_0 16-row tiles (WeightLayout::kTiled, launch.hpp).
//
// One pass at weight-load time.  Thread t writes 16-byte slot l = t % 64 of
// quant piece t / 64 = (g, p): quants 8 (l/16) .. +7 of blocks 2p and 2p+1 of
// row 16g + l % 16 (zeros for rows past N and for the block past K/32 when K/32
// is odd); the 16 threads with l < 16 also write dword l of the piece's scales.
// The tiled tensor holds every byte of the raw one once, so its traffic per
// block is the same 34 bytes; only the order changes.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}

__global__ __launch_bounds__(256) void tile_q8_0_kernel(const uint8_t* __restrict__ raw,
                                                        uint8_t* __restrict__ tiled, int N,
                                                        int KB, int KP, int64_t slots) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= slots) return;
  const int64_t piece = t >> 6;
  const int l = (int)(t & 63);
  const int64_t g = piece / KP;
  const int p = (int)(piece - g * KP);
  const int sub = l >> 4, r = l & 15;
  const int64_t row = g * kTileRows + r;
  const int64_t row_bytes = (int64_t)KB * kBlockBytes;
  uint32_t q[4] = {0u, 0u, 0u, 0u};
  uint32_t sc = 0u;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int blk = 2 * p + h;
    if (row >= N || blk >= KB) continue;
    const uint8_t* b = raw + row * row_bytes + (int64_t)blk * kBlockBytes;
    const uint8_t* qs = b + 2 + 8 * sub;  // 2-byte aligned
    q[2 * h] = ld_u16(qs) | (ld_u16(qs + 2) << 16);
    q[2 * h + 1] = ld_u16(qs + 4) | (ld_u16(qs + 6) << 16);
    sc |= ld_u16(b) << (16 * h);
  }
  *reinterpret_cast<u32x4*>(tiled + piece * kTilePieceBytes + l * 16) =
      u32x4{q[0], q[1], q[2], q[3]};
  if (sub == 0) {
    const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
    *reinterpret_cast<uint32_t*>(tiled + G * KP * kTilePieceBytes + piece * kTileScaleBytes +
                                 4 * r) = sc;
  }
}

}  // namespace

hipError_t launch_tile_q8_0(const uint8_t* raw, uint8_t* tiled, int N, int K,
                            hipStream_t stream) {
  const int KB = K / kBlockElems;
  const int KP = (KB + 1) / 2;
  const int64_t G = ((int64_t)N + kTileRows - 1) / kTileRows;
  const int64_t slots = G * KP * 64;
  const int64_t blocks = (slots + 255) / 256;
  if (N <= 0 || KB <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(tile_q8_0_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, raw, tiled,
                     N, KB, KP, slots);
  return hipGetLastError();
}

}  // namespace mle
