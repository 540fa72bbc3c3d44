"""Seeded synthetic inputs with the benchmark's value distributions (numpy, portable).

Every tensor is drawn from a counter-based SplitMix64 stream, so any slice of any tensor
can be regenerated on any machine without replaying a sequential generator:

    u64[i] = mix64(state0 + (i + 1) * GAMMA)      state0 = (seed << 8) | tag

* activations  x ~ N(0,1): Box-Muller on the pair (u64[2i], u64[2i+1]) in float64,
  cosine branch only, rounded once to float32;
* int8 quants  q = (u64[i] mod 255) - 127, i.e. uniform on [-127, 127];
* fp16 scales  d = fp16(fp32(|z| * 0.02 / 127)) with z ~ N(0,1) as above
  (about 30 % of these are binary16 subnormals, a few round to +0);
* token ids    u64[i] mod vocab.

Q8_0 weights are packed as raw GGUF ``block_q8_0`` bytes: ``[fp16 d little-endian]
[int8 q[32]]`` per 34-byte block (``include/minillm/io/gguf_format.h:42-44`` of the
reference), blocks running along the last logical dimension.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

TAG_X, TAG_Q, TAG_D, TAG_IDS, TAG_BIAS = 1, 2, 3, 4, 5
BLOCK_BYTES = 34
BLOCK_ELEMS = 32
_CHUNK = 1 << 22


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def u64_stream(seed: int, tag: int, start: int, count: int) -> np.ndarray:
    """Elements [start, start+count) of the SplitMix64 stream for (seed, tag)."""
    state0 = np.uint64(((seed << 8) | tag) & 0xFFFFFFFFFFFFFFFF)
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(state0 + i * GAMMA)


def _uniform01(u: np.ndarray) -> np.ndarray:
    return ((u >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normals64(seed: int, tag: int, start: int, count: int) -> np.ndarray:
    """float64 N(0,1) values [start, start+count) of the (seed, tag) normal stream."""
    u = u64_stream(seed, tag, 2 * start, 2 * count)
    u1 = _uniform01(u[0::2])
    u2 = _uniform01(u[1::2])
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def activations(seed: int, shape, tag: int = TAG_X) -> np.ndarray:
    """float32 activations ~ N(0,1)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        c = min(_CHUNK, n - s)
        out[s:s + c] = normals64(seed, tag, s, c).astype(np.float32)
    return out.reshape(shape)


def quants(seed: int, n: int) -> np.ndarray:
    """int8 quants uniform on [-127, 127]."""
    out = np.empty(n, dtype=np.int8)
    for s in range(0, n, _CHUNK):
        c = min(_CHUNK, n - s)
        u = u64_stream(seed, TAG_Q, s, c)
        out[s:s + c] = ((u % np.uint64(255)).astype(np.int16) - 127).astype(np.int8)
    return out


def scales_f16(seed: int, n_blocks: int) -> np.ndarray:
    """fp16 block scales d = fp16(fp32(|z| * 0.02 / 127))."""
    out = np.empty(n_blocks, dtype=np.float16)
    for s in range(0, n_blocks, _CHUNK):
        c = min(_CHUNK, n_blocks - s)
        z = normals64(seed, TAG_D, s, c)
        out[s:s + c] = (np.abs(z) * 0.02 / 127.0).astype(np.float32).astype(np.float16)
    return out


def token_ids(seed: int, count: int, vocab: int) -> np.ndarray:
    u = u64_stream(seed, TAG_IDS, 0, count)
    return (u % np.uint64(vocab)).astype(np.int32)


def pack_q8_0(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Pack int8 quants (len 32*nb) and fp16 scales (len nb) into raw Q8_0 bytes."""
    q = np.ascontiguousarray(q, dtype=np.int8).reshape(-1, BLOCK_ELEMS)
    d = np.ascontiguousarray(d, dtype=np.float16).reshape(-1)
    assert q.shape[0] == d.shape[0]
    out = np.empty((q.shape[0], BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype("<f2").view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def pack_q8_0_const_scale(q: np.ndarray, scale_bits: int) -> np.ndarray:
    """Pack with one fp16 scale for every block (the reference tests' pack_q8_0 helper).

    Values are padded with zeros up to a whole block, as the reference helper does
    (tests/test_cuda_kernels.cpp:51-65).
    """
    q = np.asarray(q, dtype=np.int8).reshape(-1)
    nb = (q.size + BLOCK_ELEMS - 1) // BLOCK_ELEMS
    qq = np.zeros(nb * BLOCK_ELEMS, dtype=np.int8)
    qq[:q.size] = q
    d = np.full(nb, scale_bits, dtype=np.uint16).view(np.float16)
    return pack_q8_0(qq, d)


def q8_0_weight(seed: int, rows: int, cols: int):
    """Raw Q8_0 bytes for a [rows, cols] weight (blocks along cols) plus (q, d)."""
    assert cols % BLOCK_ELEMS == 0
    n = rows * cols
    q = quants(seed, n)
    d = scales_f16(seed, n // BLOCK_ELEMS)
    return pack_q8_0(q, d), q, d


def dequantize(raw: np.ndarray, n_elems: int) -> np.ndarray:
    """float64 dequantisation d*q of a raw Q8_0 stream (exact: both factors fit fp64)."""
    b = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    d = b[:, 0:2].copy().view("<f2").astype(np.float64).reshape(-1, 1)
    q = b[:, 2:].view(np.int8).astype(np.float64)
    return (d * q).reshape(-1)[:n_elems]


def weight_bytes(rows: int, cols: int) -> int:
    return rows * (cols // BLOCK_ELEMS) * BLOCK_BYTES
