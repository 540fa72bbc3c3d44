// q8_0_device.hpp -- device-side helpers shared by the Q8_0 kernels (gfx950).
//
// A Q8_0 block (GGUF block_q8_0, reference include/minillm/io/gguf_format.h:42-44)
// is 34 bytes: a little-endian binary16 scale d followed by 32 int8 quants q.
// Element value = d * q.  Blocks are packed back to back, so a block starts on
// a 2-byte boundary only; all loads below are built so that they never touch a
// byte outside the 34 bytes of the block being read (no over-read past the end
// of a weight allocation).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mle {

constexpr int kBlockBytes = 34;
constexpr int kBlockElems = 32;

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Exact binary16 -> binary32 of a scale.  v_cvt_f32_f16 is exact for every
// finite input (f16 subnormals are normal f32 values; f16 denormals are kept by
// the kernel's default float mode).  NaNs are canonicalised to the default quiet
// NaN with the input's sign, which is what the reference CPU decode returns
// (src/runtime/kernels/cpu_kernels.cpp:29-31 builds quiet_NaN() then negates).
__device__ __forceinline__ float scale_to_f32(uint32_t bits16) {
  const uint16_t h = (uint16_t)bits16;
  float f = (float)__builtin_bit_cast(_Float16, h);
  const bool is_nan = ((h & 0x7c00u) == 0x7c00u) && (h & 0x3ffu);
  const uint32_t canon = ((uint32_t)(h & 0x8000u) << 16) | 0x7fc00000u;
  return is_nan ? __builtin_bit_cast(float, canon) : f;
}

// Fast decode for accumulation paths: NaN payloads are irrelevant there.
__device__ __forceinline__ float scale_to_f32_fast(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// One Q8_0 block held in registers: q[i] holds quants 4i..4i+3 (byte j of q[i]
// is quant 4i+j), and `scale_bits` the binary16 scale in its low 16 bits.
struct Block {
  uint32_t q[8];
  uint32_t scale_bits;
};

// The raw loads of one block, not yet realigned: keeping these in registers
// (instead of a Block) lets a software pipeline carry loads in flight across a
// loop iteration, since nothing touches them until the block is consumed.
struct RawBlock {
  u32x4_a4 v0, v1;  // 32 bytes from the 4-aligned address at or after the block
  uint32_t u;       // the remaining u16 (q30, q31 in case A; the scale in case B)
  uint32_t mis;     // 0 (case A) or 2 (case B)
};

// Issues the loads of the 34-byte block starting at `blk` (2-byte aligned).
//
// Case A (blk % 4 == 0): 8 dwords from blk (scale + q0..q29) and the u16 at
//   blk + 32 (q30, q31); quants are realigned by 2 bytes.
// Case B (blk % 4 == 2): 8 dwords from blk + 2 (exactly q0..q31) and the u16 at
//   blk (the scale).
// Both cases read exactly bytes [blk, blk + 34).
__device__ __forceinline__ RawBlock load_block_raw(const uint8_t* __restrict__ blk) {
  RawBlock r;
  r.mis = (uint32_t)((uintptr_t)blk & 2u);
  const uint8_t* p8 = blk + r.mis;  // 4-byte aligned
  const uint8_t* p2 = blk + (r.mis ? 0 : 32);
  r.v0 = *reinterpret_cast<const u32x4_a4*>(p8);
  r.v1 = *reinterpret_cast<const u32x4_a4*>(p8 + 16);
  r.u = *reinterpret_cast<const uint16_t*>(p2);
  return r;
}

// Realigns raw loads into quants + scale.
__device__ __forceinline__ Block finish_block(const RawBlock& r) {
  const uint32_t w[9] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w, r.v1.x, r.v1.y, r.v1.z, r.v1.w, r.u};
  const uint32_t sh = r.mis ? 0u : 2u;
  Block b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b.q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
  b.scale_bits = r.mis ? r.u : (w[0] & 0xffffu);
  return b;
}

__device__ __forceinline__ Block load_block(const uint8_t* __restrict__ blk) {
  return finish_block(load_block_raw(blk));
}

// Element n of a Linear bias: fp32, or bf16 widened exactly (the reference's
// add_bias adds weight_to_f32(bias[n]) in fp32, cuda_kernels.cu:229-233).
__device__ __forceinline__ float bias_at(const void* bias, int bf16, int64_t n) {
  if (bf16) return __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(bias)[n] << 16);
  return static_cast<const float*>(bias)[n];
}

// Cache-policy argument of the decode kernels' weight loads: non-temporal
// (gfx950 `nt`).  Each weight byte is read once per launch; streaming it past
// the caches measured 0.92-0.98x the time of plain loads on every decode kernel
// (Llama-7B shapes, MI355X), with bit-identical results.
constexpr int kNonTemporal = 2;

// Signed int8 byte j of a dword, as float (one v_cvt_f32_i32 with SDWA sext).
__device__ __forceinline__ float q_at(uint32_t word, int j) {
  return (float)(int8_t)(word >> (8 * j));
}

// Round-to-nearest-even fp32 -> bf16 of two values packed into one dword
// (lo in bits 0-15).  Inputs here are finite.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  uint32_t a = __builtin_bit_cast(uint32_t, lo);
  uint32_t b = __builtin_bit_cast(uint32_t, hi);
  a += 0x7fffu + ((a >> 16) & 1u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (a >> 16) | (b & 0xffff0000u);
}

}  // namespace mle
