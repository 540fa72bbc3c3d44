// ref_shim.cpp -- C entry points over the reference's own CPU Q8_0 kernels.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile together with
// /root/reference/src/runtime/kernels/cpu_kernels.cpp, read where it lies
// (never copied), into oracle/_ref/libref_cpu_q8_0.so.  Used only to pin the
// oracle restatement (tests/) and as the CPU baseline (bench.py).
//
// The declarations below are the reference's public signatures from
// include/minillm/runtime/kernels/cpu_kernels.h:16,21,32; they are not
// re-implemented here.
#include <cstdint>

#include "minillm/runtime/kernels/cpu_kernels.h"

extern "C" {

void ref_sgemm_nt_q8_0(const float* A, const uint8_t* W, float* C, int M, int N, int K) {
    minillm::cpu::sgemm_nt(A, W, C, M, N, K);
}

void ref_sgemm_q8_0(const float* A, const uint8_t* B, float* C, int M, int N, int K) {
    minillm::cpu::sgemm(A, B, C, M, N, K);
}

void ref_embedding_q8_0(const uint8_t* W, const int* ids, float* out, int seq_len, int hidden) {
    minillm::cpu::embedding(W, ids, out, seq_len, hidden);
}

}  // extern "C"
