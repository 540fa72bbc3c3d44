"""ctypes binding of the C ABI in ``include/mle_q8_0.h`` (``libmle_q8_0.so``).

This is plumbing for Python callers (tests, bench): device buffers come from PyTorch-ROCm
tensors, the work runs in the HIP kernels of ``libmle_q8_0.so``.  There is no fallback:
if the library is missing, every call raises.

Each wrapper accepts torch tensors (or raw integer device addresses) and the HIP stream
to launch on (default: torch's current stream).  Failures raise :class:`Q8_0Error`
carrying the reference ``ErrorCode`` value and message; the ``*_status`` variants return
``(code, message)`` instead, for error-path tests.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmle_q8_0.so")

ERROR_NAMES = {0: "Ok", 1: "InvalidArgument", 2: "OutOfRange", 3: "ShapeMismatch",
               4: "Unsupported", 5: "NotImplemented", 6: "RuntimeError"}

EXPORTED = ("mle_q8_0_abi_version", "mle_q8_0_linear", "mle_q8_0_linear_ex",
            "mle_q8_0_linear_tiled_ex",
            "mle_q8_0_linear_swiglu", "mle_q8_0_linear_multi", "mle_q8_0_matmul",
            "mle_q8_0_embedding", "mle_q8_0_embedding_tiled", "mle_argmax_f32", "mle_top_tokens_f32", "mle_swiglu_f32",
            "mle_last_error", "mle_q8_0_bytes", "mle_q8_0_f16_decode", "mle_q8_0_tiled_bytes",
            "mle_q8_0_tile", "mle_q8_0_linear_tiled", "mle_q8_0_linear_swiglu_tiled",
            "mle_q8_0_linear_multi_tiled", "mle_q8_0_workspace_size", "mle_workspace_reserve",
            "mle_workspace_info", "mle_workspace_plan_growth", "mle_q8_0_linear_noalloc",
            "mle_q8_0_dequantize", "mle_q8_0_linear_bias_bf16",
            "mle_q8_0_linear_tiled_bias_bf16", "mle_probe_stream_read")

OP_LINEAR, OP_LINEAR_SWIGLU, OP_LINEAR_MULTI, OP_MATMUL = 0, 1, 2, 3


class Q8_0Error(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


_lib = None
_vp = ctypes.c_void_p
_i = ctypes.c_int


def load() -> ctypes.CDLL:
    """Load libmle_q8_0.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m llmengine_amd.build` "
            "(there is no CPU fallback for the Q8_0 path)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.mle_q8_0_abi_version.restype = _i
    lib.mle_q8_0_abi_version.argtypes = []
    lib.mle_q8_0_linear.restype = _i
    lib.mle_q8_0_linear.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_linear_ex.restype = _i
    lib.mle_q8_0_linear_ex.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i,
                                       _vp]
    lib.mle_q8_0_linear_tiled_ex.restype = _i
    lib.mle_q8_0_linear_tiled_ex.argtypes = lib.mle_q8_0_linear_ex.argtypes
    lib.mle_q8_0_linear_swiglu.restype = _i
    lib.mle_q8_0_linear_swiglu.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_linear_multi.restype = _i
    lib.mle_q8_0_linear_multi.argtypes = [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _vp]
    lib.mle_q8_0_matmul.restype = _i
    lib.mle_q8_0_matmul.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_embedding.restype = _i
    lib.mle_q8_0_embedding.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_embedding_tiled.restype = _i
    lib.mle_q8_0_embedding_tiled.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_swiglu_f32.restype = _i
    lib.mle_swiglu_f32.argtypes = [_vp, _vp, _vp, ctypes.c_int64, _vp]
    lib.mle_probe_stream_read.restype = _i
    lib.mle_probe_stream_read.argtypes = [_vp, ctypes.c_int64, _vp, _vp]
    lib.mle_argmax_f32.restype = _i
    lib.mle_argmax_f32.argtypes = [_vp, _i, _i, _vp, _vp, _vp]
    lib.mle_top_tokens_f32.restype = _i
    lib.mle_top_tokens_f32.argtypes = [_vp, _i, _i, _i, ctypes.c_float, _vp, _vp, _vp]
    lib.mle_last_error.restype = ctypes.c_char_p
    lib.mle_last_error.argtypes = []
    lib.mle_q8_0_bytes.restype = ctypes.c_size_t
    lib.mle_q8_0_bytes.argtypes = [ctypes.c_int64]
    lib.mle_q8_0_f16_decode.restype = _i
    lib.mle_q8_0_f16_decode.argtypes = [_vp, _vp, ctypes.c_int64, _vp]
    lib.mle_q8_0_tiled_bytes.restype = ctypes.c_size_t
    lib.mle_q8_0_tiled_bytes.argtypes = [_i, _i]
    lib.mle_q8_0_tile.restype = _i
    lib.mle_q8_0_tile.argtypes = [_vp, _vp, _i, _i, _vp]
    lib.mle_q8_0_linear_tiled.restype = _i
    lib.mle_q8_0_linear_tiled.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_linear_swiglu_tiled.restype = _i
    lib.mle_q8_0_linear_swiglu_tiled.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_linear_multi_tiled.restype = _i
    lib.mle_q8_0_linear_multi_tiled.argtypes = [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _vp]
    for fn in (lib.mle_q8_0_linear_bias_bf16, lib.mle_q8_0_linear_tiled_bias_bf16):
        fn.restype = _i
        fn.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    lib.mle_q8_0_dequantize.restype = _i
    lib.mle_q8_0_dequantize.argtypes = [_vp, _vp, ctypes.c_int64, _vp]
    lib.mle_q8_0_linear_noalloc.restype = _i
    lib.mle_q8_0_linear_noalloc.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]
    _sz = ctypes.c_size_t
    lib.mle_q8_0_workspace_size.restype = _i
    lib.mle_q8_0_workspace_size.argtypes = [_i, _i, _i, _vp, _i, _i, _vp, _vp]
    lib.mle_workspace_reserve.restype = _i
    lib.mle_workspace_reserve.argtypes = [_sz, _sz, _vp]
    lib.mle_workspace_info.restype = _i
    lib.mle_workspace_info.argtypes = [_vp, _vp, _vp, _vp]
    lib.mle_workspace_plan_growth.restype = _i
    lib.mle_workspace_plan_growth.argtypes = [_sz, _sz, _sz, _sz, _vp, _vp]
    _lib = lib
    return lib


def _addr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def last_error() -> str:
    return load().mle_last_error().decode()


def _status(rc: int):
    return rc, (last_error() if rc else "")


def _raise(rc: int):
    if rc != 0:
        raise Q8_0Error(rc, last_error())


def linear_status(x, w, bias, y, M, N, K, stream=None):
    rc = load().mle_q8_0_linear(_addr(x), _addr(w), _addr(bias), _addr(y), M, N, K,
                                _stream(stream))
    return _status(rc)


def linear(x, w, bias, y, M, N, K, stream=None) -> None:
    """y[M,N] = x[M,K] . W^T (+ bias); W raw Q8_0 [N,K]."""
    _raise(linear_status(x, w, bias, y, M, N, K, stream)[0])


def linear_noalloc_status(x, w, bias, y, M, N, K, stream=None):
    rc = load().mle_q8_0_linear_noalloc(_addr(x), _addr(w), _addr(bias), _addr(y), M, N, K,
                                        _stream(stream))
    return _status(rc)


def linear_noalloc(x, w, bias, y, M, N, K, stream=None) -> None:
    """linear() with its workspace in the library's static device scratch (no
    allocation; calls overlapping on one GPU race)."""
    _raise(linear_noalloc_status(x, w, bias, y, M, N, K, stream)[0])


def linear_ex(x, w, bias, y, M, N, K, path=0, mt=0, lpr=0, rw=0, waves=0, kslice=0,
              splits=0, bm=0, bn=0, hyb=0, rpw=0, stream=None, tiled=False) -> None:
    """Linear with a forced path and launch shape (test / tuning hook).

    path 1 (FP32 GEMV) takes mt, lpr, rw, or mt and rpw (the row-span kernel on
    raw weights, rpw rows per workgroup); path 2 (MFMA GEMM) takes splits, bm, bn;
    path 3 (MFMA decode) takes mt, waves, kslice and hyb (a hybrid-kernel launch
    shape); zero = automatic.  tiled: W in 16-row tiles (path 0 or 3)."""
    if path == 3:
        t = (mt, waves or (4 if hyb else 0), kslice or (16 if hyb else 0), hyb)
    elif path == 2:
        t = (splits, bm, bn, 0)
    else:
        t = (mt, lpr or (64 if rpw else 0), rw or (1 if rpw else 0), rpw)
    fn = load().mle_q8_0_linear_tiled_ex if tiled else load().mle_q8_0_linear_ex
    rc = fn(_addr(x), _addr(w), _addr(bias), _addr(y), M, N, K, path, *t, _stream(stream))
    _raise(rc)


def linear_bias_bf16_status(x, w, bias_bf16, y, M, N, K, stream=None, tiled=False):
    fn = (load().mle_q8_0_linear_tiled_bias_bf16 if tiled else load().mle_q8_0_linear_bias_bf16)
    rc = fn(_addr(x), _addr(w), _addr(bias_bf16), _addr(y), M, N, K, _stream(stream))
    return _status(rc)


def linear_bias_bf16(x, w, bias_bf16, y, M, N, K, stream=None, tiled=False) -> None:
    """y[M,N] = x . W^T + (float)bias_bf16 (bias as raw bf16 bits, uint16 [N])."""
    _raise(linear_bias_bf16_status(x, w, bias_bf16, y, M, N, K, stream, tiled)[0])


def linear_swiglu_status(x, w_gate, w_up, y, M, N, K, stream=None):
    rc = load().mle_q8_0_linear_swiglu(_addr(x), _addr(w_gate), _addr(w_up), _addr(y), M, N,
                                       K, _stream(stream))
    return _status(rc)


def linear_swiglu(x, w_gate, w_up, y, M, N, K, stream=None) -> None:
    """y[M,N] = silu(x . Wg^T) * (x . Wu^T); Wg, Wu raw Q8_0 [N,K]."""
    _raise(linear_swiglu_status(x, w_gate, w_up, y, M, N, K, stream)[0])


def linear_multi_status(x, ws, biases, ys, Ns, M, K, stream=None, tiled=False):
    count = len(ws)
    vp_arr = _vp * max(count, 1)
    w_arr = vp_arr(*[_addr(w) for w in ws]) if ws is not None else None
    y_arr = vp_arr(*[_addr(y) for y in ys]) if ys is not None else None
    b_arr = vp_arr(*[_addr(b) for b in biases]) if biases is not None else None
    n_arr = (_i * max(count, 1))(*Ns) if Ns is not None else None
    fn = load().mle_q8_0_linear_multi_tiled if tiled else load().mle_q8_0_linear_multi
    rc = fn(_addr(x), count,
            ctypes.cast(w_arr, _vp) if w_arr else None,
            ctypes.cast(b_arr, _vp) if b_arr else None,
            ctypes.cast(y_arr, _vp) if y_arr else None,
            ctypes.cast(n_arr, _vp) if n_arr else None,
            M, K, _stream(stream))
    return _status(rc)


def linear_multi(x, ws, biases, ys, Ns, M, K, stream=None) -> None:
    """ys[i][M,Ns[i]] = x . ws[i]^T (+ biases[i]) for up to three weights, one launch."""
    _raise(linear_multi_status(x, ws, biases, ys, Ns, M, K, stream)[0])


def matmul_status(a, b, c, M, N, K, stream=None):
    rc = load().mle_q8_0_matmul(_addr(a), _addr(b), _addr(c), M, N, K, _stream(stream))
    return _status(rc)


def matmul(a, b, c, M, N, K, stream=None) -> None:
    """c[M,N] = a[M,K] . B[K,N]; B raw Q8_0 [K,N] with blocks along N."""
    _raise(matmul_status(a, b, c, M, N, K, stream)[0])


def embedding_status(w, ids, out, seq_len, vocab, hidden, stream=None):
    rc = load().mle_q8_0_embedding(_addr(w), _addr(ids), _addr(out), seq_len, vocab,
                                   hidden, _stream(stream))
    return _status(rc)


def embedding(w, ids, out, seq_len, vocab, hidden, stream=None) -> None:
    """out[s,h] = dequantised row ids[s] of a raw Q8_0 [vocab, hidden] table."""
    _raise(embedding_status(w, ids, out, seq_len, vocab, hidden, stream)[0])


def embedding_tiled_status(w_tiled, ids, out, seq_len, vocab, hidden, stream=None):
    rc = load().mle_q8_0_embedding_tiled(_addr(w_tiled), _addr(ids), _addr(out), seq_len,
                                         vocab, hidden, _stream(stream))
    return _status(rc)


def embedding_tiled(w_tiled, ids, out, seq_len, vocab, hidden, stream=None) -> None:
    """The embedding gather from a table in 16-row tiles (mle_q8_0_tile of [vocab, hidden])."""
    _raise(embedding_tiled_status(w_tiled, ids, out, seq_len, vocab, hidden, stream)[0])


def swiglu_status(gate, up, y, n, stream=None):
    rc = load().mle_swiglu_f32(_addr(gate), _addr(up), _addr(y), n, _stream(stream))
    return _status(rc)


def swiglu(gate, up, y, n, stream=None) -> None:
    """y[i] = silu(gate[i]) * up[i] for n fp32 elements."""
    _raise(swiglu_status(gate, up, y, n, stream)[0])


def probe_stream_read_status(src, nbytes, sink, stream=None):
    rc = load().mle_probe_stream_read(_addr(src), nbytes, _addr(sink), _stream(stream))
    return _status(rc)


def probe_stream_read(src, nbytes, sink, stream=None) -> None:
    """Reads nbytes of src once (a measurement aid: the pure-read time of a buffer)."""
    _raise(probe_stream_read_status(src, nbytes, sink, stream)[0])


def argmax_status(logits, rows, n, idx, val=None, stream=None):
    rc = load().mle_argmax_f32(_addr(logits), rows, n, _addr(idx), _addr(val), _stream(stream))
    return _status(rc)


def argmax(logits, rows, n, idx, val=None, stream=None) -> None:
    """idx[r] (int32) = first index of the maximum of logits row r; val[r] its value."""
    _raise(argmax_status(logits, rows, n, idx, val, stream)[0])


def top_tokens_status(logits, rows, n, top_n, ids, probs, temperature=1.0, stream=None):
    rc = load().mle_top_tokens_f32(_addr(logits), rows, n, top_n, float(temperature),
                                   _addr(ids), _addr(probs), _stream(stream))
    return _status(rc)


def top_tokens(logits, rows, n, top_n, ids, probs, temperature=1.0, stream=None) -> None:
    """ids/probs [rows, min(top_n, n)]: the top tokens of each logits row by softmax
    probability (after 1/temperature), largest first (Sampler::get_top_tokens)."""
    _raise(top_tokens_status(logits, rows, n, top_n, ids, probs, temperature, stream)[0])


def dequantize_status(src, dst, n, stream=None):
    rc = load().mle_q8_0_dequantize(_addr(src), _addr(dst), n, _stream(stream))
    return _status(rc)


def dequantize(src, dst, n, stream=None) -> None:
    """dst[e] = q * d for the n elements of a raw Q8_0 block stream."""
    _raise(dequantize_status(src, dst, n, stream)[0])


def f16_decode(bits, out, n, stream=None) -> None:
    _raise(load().mle_q8_0_f16_decode(_addr(bits), _addr(out), n, _stream(stream)))


def q8_0_bytes(numel: int) -> int:
    return load().mle_q8_0_bytes(numel)


# Q8_0 16-row tiles: the raw bytes reordered once at load time (layout in
# include/mle_q8_0.h); the *_tiled entry points take weights in that layout.

def tiled_bytes(N: int, K: int) -> int:
    return load().mle_q8_0_tiled_bytes(N, K)


def tile_status(w, w_tiled, N, K, stream=None):
    rc = load().mle_q8_0_tile(_addr(w), _addr(w_tiled), N, K, _stream(stream))
    return _status(rc)


def tile(w, w_tiled, N, K, stream=None) -> None:
    """w_tiled = the 16-row tiled form of the raw Q8_0 weight w [N,K]."""
    _raise(tile_status(w, w_tiled, N, K, stream)[0])


def linear_tiled_status(x, w_tiled, bias, y, M, N, K, stream=None):
    rc = load().mle_q8_0_linear_tiled(_addr(x), _addr(w_tiled), _addr(bias), _addr(y), M, N,
                                      K, _stream(stream))
    return _status(rc)


def linear_tiled(x, w_tiled, bias, y, M, N, K, stream=None) -> None:
    """linear() on a tiled weight."""
    _raise(linear_tiled_status(x, w_tiled, bias, y, M, N, K, stream)[0])


def linear_swiglu_tiled_status(x, w_gate, w_up, y, M, N, K, stream=None):
    rc = load().mle_q8_0_linear_swiglu_tiled(_addr(x), _addr(w_gate), _addr(w_up), _addr(y),
                                             M, N, K, _stream(stream))
    return _status(rc)


def linear_swiglu_tiled(x, w_gate, w_up, y, M, N, K, stream=None) -> None:
    """linear_swiglu() on tiled weights."""
    _raise(linear_swiglu_tiled_status(x, w_gate, w_up, y, M, N, K, stream)[0])


def linear_multi_tiled(x, ws, biases, ys, Ns, M, K, stream=None) -> None:
    """linear_multi() on tiled weights."""
    _raise(linear_multi_status(x, ws, biases, ys, Ns, M, K, stream, tiled=True)[0])


# Workspace reservation (include/mle_q8_0.h): sizes a call would use, reserving
# them ahead of the hot path, and the per-stream workspace's capacity.

def workspace_size_status(op, M, Ns, K, tiled=False):
    """(code, message, bytes, counters) of the workspace an op would use."""
    n_arr = (_i * max(len(Ns), 1))(*Ns)
    b, c = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = load().mle_q8_0_workspace_size(op, M, len(Ns), ctypes.cast(n_arr, _vp), K,
                                        1 if tiled else 0, ctypes.byref(b), ctypes.byref(c))
    code, msg = _status(rc)
    return code, msg, b.value, c.value


def workspace_size(op, M, Ns, K, tiled=False):
    code, msg, b, c = workspace_size_status(op, M, Ns, K, tiled)
    _raise(code)
    return b, c


def workspace_reserve(nbytes, counters, stream=None) -> None:
    _raise(load().mle_workspace_reserve(nbytes, counters, _stream(stream)))


def workspace_info(stream=None):
    """(bytes, counters, generation) of the (current device, stream) workspace."""
    b, c, g = ctypes.c_size_t(0), ctypes.c_size_t(0), ctypes.c_uint64(0)
    _raise(load().mle_workspace_info(_stream(stream), ctypes.byref(b), ctypes.byref(c),
                                     ctypes.byref(g)))
    return b.value, c.value, g.value


def workspace_plan_growth(cap_bytes, cap_counters, need_bytes, need_counters):
    """(grow, new_bytes, new_counters) under the library's growth rule."""
    nb, nc = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = load().mle_workspace_plan_growth(cap_bytes, cap_counters, need_bytes, need_counters,
                                          ctypes.byref(nb), ctypes.byref(nc))
    return bool(rc), nb.value, nc.value
