// embedding.hip -- Q8_0 Embedding gather-dequantise for gfx950.
//
// out[s, h] = d * q of element h of table row ids[s]; an id outside [0, vocab)
// gives a row of +0.0f (device semantics of the reference,
// src/runtime/kernels/cuda_kernels.cu:399-427; the host adapter of the CPU path
// instead rejects such ids, cpu_kernel_adapter.cpp:72-78).
//
// HBM-bound on the fp32 writes: per token 4*hidden bytes written against
// 34*hidden/32 read.  One thread writes 4 consecutive outputs as one 16-byte
// store, so a wavefront writes 1 KiB contiguous; the 8 threads that share a
// block read its scale and quants through L1 with 2-byte loads that never
// leave the 34 bytes of the block.  The value is one fp32 multiply d*q, the
// same single rounding as the reference CPU kernel (cpu_kernels.cpp:45-51), so
// the output is bit-identical to it.
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
  *reinterpret_cast<f32x4*>(out + s * hidden + h) = v;
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

hipError_t launch_f16_decode(const uint16_t* bits, float* out, int64_t n,
                             hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(f16_decode_kernel, dim3((unsigned)((n + 255) / 256)),
                     dim3(256), 0, stream, bits, out, n);
  return hipGetLastError();
}

}  // namespace mle
