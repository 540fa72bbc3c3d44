/*
 * q8_0_oracle.c -- CPU oracle for the Q8_0 weight-only Linear / MatMul /
 * Embedding path of MiniLLMEngine (plutoaac/llmengine).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (llmengine_amd/, include/)
 * links, loads or calls this file.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker / the CPU
 * baseline, never as the thing measured or shipped.
 *
 * This is a restatement, written from the arithmetic, of the reference CPU
 * kernels.  Every function keeps the reference's exact rounding sequence so
 * that its outputs are bit-identical to the reference built with its own flags
 * (-O3, FMA contraction on, OpenMP):
 *
 *   element value   v = d * (float)q           one fp32 rounding
 *   dot product     acc = fma(x[k], v, acc)    k ascending, acc starts at +0.0f
 *
 * Parity pins (all in tests/): bit-exact against the reference's own
 * cpu_kernels.cpp compiled into oracle/_ref (where /root/reference exists),
 * against the golden fixtures under tests/golden/, against closed forms
 * (exhaustive binary16 decode vs numpy.float16, exact integer-valued known
 * answers from the reference tests) and against an FP64 brute force.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define Q8_BLOCK_BYTES 34 /* include/minillm/io/gguf_format.h:43 */
#define Q8_BLOCK_ELEMS 32 /* include/minillm/io/gguf_format.h:44 */

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/*
 * IEEE binary16 -> binary32, exact.  Follows
 * src/runtime/kernels/cpu_kernels.cpp:21-37: subnormals are mant * 2^-24,
 * Inf keeps its sign, every NaN becomes the default quiet NaN with the input's
 * sign (the reference builds quiet_NaN() and then negates it).
 */
float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* 0 or subnormal: mant * 2^-24 (exact: mant < 2^10, power-of-two scale) */
        const float mag = (float)m * 0x1p-24f;
        return bits_f32(f32_bits(mag) | sign);
    }
    if (e == 31) {
        return bits_f32(sign | (m == 0 ? 0x7f800000u : 0x7fc00000u));
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* Little-endian u16 scale at block bytes 0-1: cpu_kernels.cpp:39-43. */
static inline float block_scale(const uint8_t* block) {
    return oracle_f16_to_f32((uint16_t)(block[0] | ((uint16_t)block[1] << 8)));
}

/*
 * Value of flat element e of a Q8_0 stream: block e/32, offset e%32,
 * d * (float)q with one rounding.  cpu_kernels.cpp:45-51.
 */
static inline float q8_value(const uint8_t* blocks, size_t e) {
    const uint8_t* block = blocks + (e / Q8_BLOCK_ELEMS) * Q8_BLOCK_BYTES;
    const int8_t q = (int8_t)block[2 + e % Q8_BLOCK_ELEMS];
    return block_scale(block) * (float)q;
}

/*
 * Linear: C[M,N] = A[M,K] . W^T, W row n is the contiguous Q8_0 stream
 * starting at element n*K.  cpu_kernels.cpp:208-218 (OpenMP over m only) with
 * the dot product of cpu_kernels.cpp:53-60 (acc += a*v, contracted to fma).
 */
void oracle_sgemm_nt_q8_0(const float* A, const uint8_t* W, float* C,
                          int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const float* a = A + (size_t)m * K;
        float* c = C + (size_t)m * N;
        for (int n = 0; n < N; ++n) {
            const size_t base = (size_t)n * K;
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) {
                acc = fmaf(a[k], q8_value(W, base + (size_t)k), acc);
            }
            c[n] = acc;
        }
    }
}

/*
 * MatMul: C[M,N] = A[M,K] . B[K,N], element (k,n) is flat index k*N+n of the
 * Q8_0 stream, so blocks run along N.  cpu_kernels.cpp:116-130 (OpenMP over m
 * only, acc += a*v contracted to fma, k ascending).
 */
void oracle_sgemm_q8_0(const float* A, const uint8_t* B, float* C,
                       int M, int N, int K) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const float* a = A + (size_t)m * K;
        float* c = C + (size_t)m * N;
        for (int n = 0; n < N; ++n) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) {
                acc = fmaf(a[k], q8_value(B, (size_t)k * N + n), acc);
            }
            c[n] = acc;
        }
    }
}

/*
 * Embedding: out[s,h] = value of element ids[s]*hidden + h.
 * cpu_kernels.cpp:286-295 (single-threaded; ids are range-checked by the
 * caller, src/runtime/kernels/cpu_kernel_adapter.cpp:72-78).
 */
void oracle_embedding_q8_0(const uint8_t* W, const int32_t* ids, float* out,
                           int seq_len, int hidden) {
    for (int s = 0; s < seq_len; ++s) {
        const size_t row = (size_t)ids[s] * (size_t)hidden;
        float* o = out + (size_t)s * hidden;
        for (int h = 0; h < hidden; ++h) o[h] = q8_value(W, row + (size_t)h);
    }
}

/*
 * Device-side embedding semantics: an id outside [0, vocab) yields a row of
 * +0.0f instead of an error, because the device path cannot range-check ids
 * on the host (src/runtime/kernels/cuda_kernels.cu:410-415).  Valid ids follow
 * oracle_embedding_q8_0 exactly.
 */
void oracle_embedding_q8_0_zero_fill(const uint8_t* W, const int32_t* ids,
                                     float* out, int seq_len, int vocab,
                                     int hidden) {
    for (int s = 0; s < seq_len; ++s) {
        float* o = out + (size_t)s * hidden;
        const int32_t id = ids[s];
        if (id < 0 || id >= vocab) {
            for (int h = 0; h < hidden; ++h) o[h] = 0.0f;
            continue;
        }
        const size_t row = (size_t)id * (size_t)hidden;
        for (int h = 0; h < hidden; ++h) o[h] = q8_value(W, row + (size_t)h);
    }
}

/* Linear bias epilogue: y[m,n] += bias[n], cpu_kernel_adapter.cpp:126-140. */
void oracle_add_bias(float* Y, const float* bias, int M, int N) {
    for (int m = 0; m < M; ++m) {
        float* y = Y + (size_t)m * N;
        for (int n = 0; n < N; ++n) y[n] = y[n] + bias[n];
    }
}

/* Whole-stream dequantisation (gguf_weight_loader.cpp:446-463 semantics). */
void oracle_dequantize_q8_0(const uint8_t* W, float* out, size_t n_elems) {
    for (size_t e = 0; e < n_elems; ++e) out[e] = q8_value(W, e);
}
