// embedding.hip -- Q8_0 Embedding gather-dequantise for gfx950 (from raw GGUF
// blocks or from 16-row tiles), and the whole-tensor Q8_0 -> fp32
// dequantisation of the weight loader.
//
// out[s, h] = d * q of element h of table row ids[s]; an id outside [0, vocab)
// gives a row of +0.0f (device semantics of the reference,
// src/runtime/kernels/cuda_kernels.cu:399-427; the host adapter of the CPU path
// instead rejects such ids, cpu_kernel_adapter.cpp:72-78).
//
// HBM-bound on the fp32 writes: per token 4*hidden bytes written against
// 34*hidden/32 read.  One thread writes 4 consecutive outputs as one 16-byte
// non-temporal store (the output is not read back by this kernel, so it goes
// to memory without displacing the table's lines in L2: 17% faster than plain
// stores on the configs[4] gather, MI355X), so a wavefront writes 1 KiB
// contiguous; the 8 threads that share a block read its scale and quants
// through L1 with 2-byte loads that never leave the 34 bytes of the block.  The
// value is one fp32 multiply d*q, the same single rounding as the reference CPU
// kernel (cpu_kernels.cpp:45-51), so the output is bit-identical to it.
//
// dequantize_q8_0_kernel: dst[e] = q * d for the flat element stream of a Q8_0
// tensor (WeightLoader::dequantize_to_f32, Q8_0 case,
// src/io/gguf_weight_loader.cpp:446-463): the same single fp32 multiply, with
// the loader's binary16 decode (exact; NaN quieted with its sign, as
// scale_to_f32), so the bits equal the host loop's.
#include "../launch.hpp"
#include "../q8_0_device.hpp"

namespace mle {
namespace {

__global__ __launch_bounds__(256) void embedding_q8_0_kernel(
    const uint8_t* __restrict__ w, const int32_t* __restrict__ ids,
    float* __restrict__ out, int64_t total_quads, int quads_per_row, int vocab,
    int hidden) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total_quads) return;
  const int64_t s = g / quads_per_row;
  const int h = (int)(g - s * quads_per_row) * 4;
  const int32_t id = ids[s];
  f32x4 v;
  if (id < 0 || id >= vocab) {
    v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  } else {
    const int64_t blocks_per_row = hidden / kBlockElems;
    const uint8_t* blk =
        w + ((int64_t)id * blocks_per_row + h / kBlockElems) * kBlockBytes;
    const uint16_t* hp = reinterpret_cast<const uint16_t*>(blk);
    const int o = (h % kBlockElems) / 2;  // quants h, h+1 are u16 number 1 + o of the block
    const uint32_t sbits = hp[0];
    const uint32_t lo = hp[1 + o];
    const uint32_t hi = hp[2 + o];
    const float d = scale_to_f32(sbits);
    const uint32_t q = lo | (hi << 16);
    v.x = d * q_at(q, 0);
    v.y = d * q_at(q, 1);
    v.z = d * q_at(q, 2);
    v.w = d * q_at(q, 3);
  }
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + s * hidden + h));
}

// The same gather from a table in Q8_0 16-row tiles (layout of launch.hpp):
// element h of row n sits in quant piece (n / 16, pair h / 64), slot
// 16 ((h % 32) / 8) + n % 16, byte 8 ((h / 32) % 2) + h % 8, and its scale in
// dword n % 16 of the matching scale piece (low half: even block, high half: odd
// block).  Four consecutive outputs are one aligned dword of quants.  Same value
// d * q with the same decode, so the output equals the raw gather bit for bit.
__global__ __launch_bounds__(256) void embedding_q8_0_tiled_kernel(
    const uint8_t* __restrict__ w, const int32_t* __restrict__ ids,
    float* __restrict__ out, int64_t total_quads, int quads_per_row, int vocab,
    int hidden) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= total_quads) return;
  const int64_t s = g / quads_per_row;
  const int h = (int)(g - s * quads_per_row) * 4;
  const int32_t id = ids[s];
  f32x4 v;
  if (id < 0 || id >= vocab) {
    v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  } else {
    const int64_t KP = (hidden / kBlockElems + 1) / 2;
    const int64_t G = ((int64_t)vocab + kTileRows - 1) / kTileRows;
    const int64_t piece = (int64_t)(id / kTileRows) * KP + h / (2 * kBlockElems);
    const int r = id % kTileRows, e = h % kBlockElems, odd = (h / kBlockElems) & 1;
    const uint32_t q = *reinterpret_cast<const uint32_t*>(
        w + piece * kTilePieceBytes + (16 * (e / 8) + r) * 16 + 8 * odd + e % 8);
    const uint32_t sc = *reinterpret_cast<const uint32_t*>(
        w + G * KP * kTilePieceBytes + piece * kTileScaleBytes + r * 4);
    const float d = scale_to_f32(odd ? sc >> 16 : sc & 0xffffu);
    v.x = d * q_at(q, 0);
    v.y = d * q_at(q, 1);
    v.z = d * q_at(q, 2);
    v.w = d * q_at(q, 3);
  }
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + s * hidden + h));
}

__global__ __launch_bounds__(256) void dequantize_q8_0_kernel(const uint8_t* __restrict__ w,
                                                              float* __restrict__ out,
                                                              int64_t n) {
  const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (e >= n) return;
  const uint16_t* hp = reinterpret_cast<const uint16_t*>(w + (e / kBlockElems) * kBlockBytes);
  const int o = (int)(e % kBlockElems) / 2;  // quants e, e+1 are u16 number 1 + o of the block
  const float d = scale_to_f32(hp[0]);
  if (e + 4 <= n) {
    const uint32_t q = (uint32_t)hp[1 + o] | ((uint32_t)hp[2 + o] << 16);
    const f32x4 v = {q_at(q, 0) * d, q_at(q, 1) * d, q_at(q, 2) * d, q_at(q, 3) * d};
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(out + e));
    return;
  }
  // Tail of a tensor whose element count is not a multiple of 4: the bytes past
  // the last element of its (partial) last block are not read.
  const int8_t* qs = reinterpret_cast<const int8_t*>(hp + 1) + (e % kBlockElems);
  for (int64_t i = 0; e + i < n; ++i) out[e + i] = (float)qs[i] * d;
}

__global__ __launch_bounds__(256) void f16_decode_kernel(
    const uint16_t* __restrict__ bits, float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = scale_to_f32(bits[i]);
}

}  // namespace

hipError_t launch_embedding(const uint8_t* w, const int32_t* ids, float* out,
                            int64_t seq_len, int vocab, int hidden,
                            hipStream_t stream) {
  const int quads_per_row = hidden / 4;
  const int64_t total = seq_len * quads_per_row;
  if (total == 0) return hipSuccess;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(embedding_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0,
                     stream, w, ids, out, total, quads_per_row, vocab, hidden);
  return hipGetLastError();
}

hipError_t launch_embedding_tiled(const uint8_t* w, const int32_t* ids, float* out,
                                  int64_t seq_len, int vocab, int hidden, hipStream_t stream) {
  const int quads_per_row = hidden / 4;
  const int64_t total = seq_len * quads_per_row;
  if (total == 0) return hipSuccess;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(embedding_q8_0_tiled_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                     w, ids, out, total, quads_per_row, vocab, hidden);
  return hipGetLastError();
}

hipError_t launch_dequantize_q8_0(const uint8_t* w, float* out, int64_t n,
                                  hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t grid = ((n + 3) / 4 + 255) / 256;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dequantize_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, stream, w, out,
                     n);
  return hipGetLastError();
}

hipError_t launch_f16_decode(const uint16_t* bits, float* out, int64_t n,
                             hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(f16_decode_kernel, dim3((unsigned)((n + 255) / 256)),
                     dim3(256), 0, stream, bits, out, n);
  return hipGetLastError();
}

}  // namespace mle
