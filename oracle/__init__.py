"""CPU oracle for the Q8_0 Linear / MatMul / Embedding path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker or the timed CPU baseline.  The product
(``llmengine_amd``) never imports it.

Two CPU implementations are exposed through ctypes:

* ``liboracle_q8_0.so`` -- ``q8_0_oracle.c``, a restatement of the reference kernels
  (``src/runtime/kernels/cpu_kernels.cpp:21-60,116-130,208-218,286-295``).
* ``_ref/libref_cpu_q8_0.so`` -- the reference's own ``cpu_kernels.cpp`` compiled from
  ``/root/reference`` by ``oracle/Makefile``.  It exists only where it was built.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle_q8_0.so")
REF_SO = os.path.join(HERE, "_ref", "libref_cpu_q8_0.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_int = ctypes.c_int


def _ptr(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


class _Lib:
    def __init__(self, path: str, prefix: str):
        self.path = path
        self.lib = ctypes.CDLL(path)
        self.prefix = prefix
        for name in ("sgemm_nt_q8_0", "sgemm_q8_0"):
            fn = getattr(self.lib, prefix + name)
            fn.argtypes = [_f32p, _u8p, _f32p, _int, _int, _int]
            fn.restype = None
        fn = getattr(self.lib, prefix + "embedding_q8_0")
        fn.argtypes = [_u8p, _i32p, _f32p, _int, _int]
        fn.restype = None

    def sgemm_nt(self, A: np.ndarray, W: np.ndarray, M: int, N: int, K: int) -> np.ndarray:
        """Linear ``C = A . W^T`` with W as raw Q8_0 bytes ([N,K], blocks along K)."""
        A = np.ascontiguousarray(A, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.uint8)
        assert A.size >= M * K and W.size >= N * (K // 32) * 34
        C = np.empty((M, N), dtype=np.float32)
        getattr(self.lib, self.prefix + "sgemm_nt_q8_0")(
            _ptr(A, _f32p), _ptr(W, _u8p), _ptr(C, _f32p), M, N, K)
        return C

    def sgemm(self, A: np.ndarray, B: np.ndarray, M: int, N: int, K: int) -> np.ndarray:
        """MatMul ``C = A . B`` with B as raw Q8_0 bytes ([K,N], blocks along N)."""
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.uint8)
        assert A.size >= M * K and B.size >= (K * N // 32) * 34
        C = np.empty((M, N), dtype=np.float32)
        getattr(self.lib, self.prefix + "sgemm_q8_0")(
            _ptr(A, _f32p), _ptr(B, _u8p), _ptr(C, _f32p), M, N, K)
        return C

    def embedding(self, W: np.ndarray, ids: np.ndarray, hidden: int) -> np.ndarray:
        """Gather-dequantise rows ``ids`` of a Q8_0 table with ``hidden`` columns."""
        W = np.ascontiguousarray(W, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        out = np.empty((ids.size, hidden), dtype=np.float32)
        getattr(self.lib, self.prefix + "embedding_q8_0")(
            _ptr(W, _u8p), _ptr(ids, _i32p), _ptr(out, _f32p), ids.size, hidden)
        return out


class Oracle(_Lib):
    """The C restatement (always available once ``make -C oracle`` has run)."""

    def __init__(self):
        super().__init__(ORACLE_SO, "oracle_")
        self.lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        self.lib.oracle_f16_to_f32.restype = ctypes.c_float
        self.lib.oracle_embedding_q8_0_zero_fill.argtypes = [_u8p, _i32p, _f32p, _int, _int, _int]
        self.lib.oracle_embedding_q8_0_zero_fill.restype = None
        self.lib.oracle_add_bias.argtypes = [_f32p, _f32p, _int, _int]
        self.lib.oracle_add_bias.restype = None
        self.lib.oracle_dequantize_q8_0.argtypes = [_u8p, _f32p, ctypes.c_size_t]
        self.lib.oracle_dequantize_q8_0.restype = None

    def f16_to_f32(self, bits: int) -> float:
        return self.lib.oracle_f16_to_f32(bits)

    def f16_table(self) -> np.ndarray:
        """Decode of all 65536 binary16 patterns, as float32."""
        return np.array([self.lib.oracle_f16_to_f32(i) for i in range(65536)], dtype=np.float32)

    def embedding_zero_fill(self, W: np.ndarray, ids: np.ndarray, vocab: int, hidden: int) -> np.ndarray:
        """Device semantics: ids outside [0, vocab) give rows of +0.0f."""
        W = np.ascontiguousarray(W, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        out = np.empty((ids.size, hidden), dtype=np.float32)
        self.lib.oracle_embedding_q8_0_zero_fill(
            _ptr(W, _u8p), _ptr(ids, _i32p), _ptr(out, _f32p), ids.size, vocab, hidden)
        return out

    def dequantize_q8_0(self, W: np.ndarray, n: int) -> np.ndarray:
        """The n elements of a raw Q8_0 block stream as fp32 (the weight loader's
        dequantize_to_f32, gguf_weight_loader.cpp:446-463)."""
        W = np.ascontiguousarray(W, dtype=np.uint8)
        assert W.size >= (n + 31) // 32 * 34
        out = np.empty(n, dtype=np.float32)
        self.lib.oracle_dequantize_q8_0(_ptr(W, _u8p), _ptr(out, _f32p), n)
        return out

    def linear(self, A, W, bias, M, N, K):
        """Linear with optional bias epilogue (cpu_kernel_adapter.cpp:92-142)."""
        C = self.sgemm_nt(A, W, M, N, K)
        if bias is not None:
            b = np.ascontiguousarray(bias, dtype=np.float32)
            self.lib.oracle_add_bias(_ptr(C, _f32p), _ptr(b, _f32p), M, N)
        return C


class Reference(_Lib):
    """The reference's own cpu_kernels.cpp (only where oracle/_ref was built)."""

    def __init__(self):
        super().__init__(REF_SO, "ref_")


_oracle = None


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run make -C oracle)")
        _oracle = Oracle()
    return _oracle


def reference_available() -> bool:
    return os.path.exists(REF_SO)


def reference() -> Reference:
    return Reference()
