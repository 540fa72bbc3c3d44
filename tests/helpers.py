"""Helpers shared by the GPU tests: host<->device copies and error metrics."""
from __future__ import annotations

import hashlib
import sys

import numpy as np


def note(msg: str) -> None:
    """Print the case about to run (flushed) so a failing GPU step names itself."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def empty_f32(shape, dev):
    import torch
    # filled with NaN so that an output the kernel forgets to write fails the check
    return torch.full(shape, float("nan"), dtype=torch.float32, device=dev)


def to_host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def rel_l2(a, ref) -> float:
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(a - ref) / (den if den > 0 else 1.0))


def rows_decode(M, N, K):
    """The C ABI's choice of the row-range MFMA decode for a tiled single-output
    Linear (mle::decode_mfma_pick): K 2048-4096 in steps of 64, and 3-8 tokens on
    512-1024 16-row groups or 3-4 tokens on 240-256 groups (M = 5 keeps the
    split-K kernel's 5-token tile)."""
    G = (N + 15) // 16
    if K % 64 != 0 or not 2048 <= K <= 4096:
        return False
    four = M in (3, 4)
    return ((four or 6 <= M <= 8) and 512 <= G <= 1024) or (four and 240 <= G <= 256)


def rows_decode_raw(M, N, K):
    """The C ABI's choice of the row-range MFMA decode for a raw single- or
    multi-output Linear (N = all outputs' rows): 3-4 tokens on 512-1024 16-row
    groups, K 2048-4096 in steps of 64."""
    G = (N + 15) // 16
    return M in (3, 4) and 512 <= G <= 1024 and K % 64 == 0 and 2048 <= K <= 4096


def hybrid_decode(M, N, K):
    """The C ABI's choice of the hybrid MFMA decode (row groups x a short K split)
    for a tiled plain Linear (mle::decode_mfma_pick): 3-4 or 6-8 tokens, rows of
    8192+ elements in at most 8 splits of 44 blocks, at most 256 16-row groups."""
    G = (N + 15) // 16
    return (M in (3, 4) or 6 <= M <= 8) and K >= 8192 and K // 32 <= 8 * 44 and G <= 256


def rows_decode_swiglu(M, N, K):
    """The C ABI's choice of the row-range MFMA decode for a tiled gate/up SwiGLU
    launch (mle::decode_mfma_pick_segs): K 2048-4096 in steps of 64, 3-4 or 6-8
    tokens, 512-1024 16-row groups per weight."""
    G = (N + 15) // 16
    if K % 64 != 0 or not 2048 <= K <= 4096:
        return False
    return (M in (3, 4) or 6 <= M <= 8) and 512 <= G <= 1024


def rows_decode_multi(M, Ns, K):
    """rows_decode for a tiled multi-output Linear: the outputs' 16-row groups
    (each output rounded up to whole groups) counted together."""
    G = sum((n + 15) // 16 for n in Ns)
    return rows_decode(M, 16 * G, K)


def assert_bitexact(got, want, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    diff = np.nonzero(bits(got)[~wn] != bits(want)[~wn])[0]
    assert diff.size == 0, f"{what}: {diff.size} values differ, first at {diff[:5]}"


# ---------------------------------------------------------------------------
# Q8_0 16-row tiles (layout of mle_q8_0_tile, include/mle_q8_0.h), restated in
# numpy as the checker of the device repack.

def tiled_shape(N: int, K: int):
    KB = K // 32
    return KB, (KB + 1) // 2, (N + 15) // 16


def tile_ref(raw: np.ndarray, N: int, K: int) -> np.ndarray:
    """Raw Q8_0 bytes of W[N,K] -> tiled bytes (quant pieces, then scale pieces)."""
    KB, KP, G = tiled_shape(N, K)
    blocks = np.asarray(raw, np.uint8).reshape(N, KB, 34)
    q = np.zeros((G * 16, 2 * KP, 32), np.uint8)
    d = np.zeros((G * 16, 2 * KP, 2), np.uint8)
    q[:N, :KB] = blocks[:, :, 2:]
    d[:N, :KB] = blocks[:, :, :2]
    # piece (g, p), slot 16 sub + r, half h: quants 8 sub .. of block 2p+h, row 16g+r
    qt = q.reshape(G, 16, KP, 2, 4, 8).transpose(0, 2, 4, 1, 3, 5).reshape(-1)
    # piece (g, p), dword r: scale bytes of block 2p, then 2p+1, of row 16g+r
    dt = d.reshape(G, 16, KP, 2, 2).transpose(0, 2, 1, 3, 4).reshape(-1)
    return np.concatenate([qt, dt])


def untile_ref(tiled: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of tile_ref (drops the zero padding)."""
    KB, KP, G = tiled_shape(N, K)
    t = np.asarray(tiled, np.uint8)
    nq = G * KP * 1024
    q = t[:nq].reshape(G, KP, 4, 16, 2, 8).transpose(0, 3, 1, 4, 2, 5).reshape(G * 16, 2 * KP, 32)
    d = t[nq:].reshape(G, KP, 16, 2, 2).transpose(0, 2, 1, 3, 4).reshape(G * 16, 2 * KP, 2)
    out = np.concatenate([d[:N, :KB], q[:N, :KB]], axis=2)
    return out.reshape(-1)
