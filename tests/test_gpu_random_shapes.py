"""GPU parity over a seeded sweep of Linear shapes through the automatic path choice.

Every kernel the C ABI can pick for a Linear (FP32 GEMV and its row-span variant, the
tiled FP32 GEMV, the split-K / row-range / hybrid MFMA decode, the bf16 MFMA GEMM) is
reached by some case of a fixed list of random shapes: 1-130 tokens, ragged output
counts, rows of 1-400 blocks, with and without bias, on raw and on tiled weights.
Each output is checked on sampled rows against the CPU oracle (reference
cpu_kernels.cpp:208-218) at the path's bar (relative L2 1e-5 below 64 tokens, 1e-2 on
the bf16 GEMM), and the tiled launch against the raw one (1e-6 below 64 tokens: the
same exact block products, at most grouped differently over K; 1e-2 on the GEMM, whose
two layouts round the same bf16 operands).  Every output element must be written (the
outputs start as NaN).
"""
import numpy as np
import pytest

from helpers import empty_f32, note, rel_l2, to_dev, to_host
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _cases(n=36, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.choice([1, 1, 2, 3, 4, 4, 5, 6, 7, 8, 8, 11, 16, 23, 64, 77, 130]))
        N = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 5000)),
                            int(rng.integers(5000, 17000))]))
        KB = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(40, 140)),
                             int(rng.integers(140, 400))]))
        bias = bool(rng.integers(0, 2))
        out.append((i, M, N, 32 * KB, bias))
    return out


# Fixed additions so every launch rule is reached whatever the draw: raw row-range at
# 3-4 tokens (512-1024 row groups), hybrid at 7 tokens, the one-token row-span kernel
# just past 4096-element rows.
CASES = _cases() + [(36, 4, 9000, 3008, True), (37, 3, 16000, 2048, False),
                    (38, 7, 4000, 9664, True), (39, 1, 4096, 4128, True)]


def test_sweep_reaches_the_kernel_families():
    """The fixed list spans one token, 2-63 tokens on short and long rows, and the GEMM."""
    Ms = {c[1] for c in CASES}
    assert 1 in Ms and any(2 <= m <= 8 for m in Ms) and any(m >= 64 for m in Ms)
    assert any(c[3] > 4096 for c in CASES) and any(c[3] <= 1024 for c in CASES)
    assert any(c[2] > 8192 for c in CASES)


@pytest.mark.parametrize("i,M,N,K,bias", CASES)
def test_random_linear_shapes(dev, orc, i, M, N, K, bias):
    import torch
    note(f"random shape #{i}: M={M} N={N} K={K} bias={bias}")
    w = S.q8_0_weight(700 + i, N, K)[0]
    x = S.activations(800 + i, (M, K))
    b = S.activations(900 + i, (N,), tag=S.TAG_BIAS) if bias else None
    dx, dw = to_dev(x, dev), to_dev(w, dev)
    db = to_dev(b, dev) if bias else None
    dt = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
    capi.tile(dw, dt, N, K)
    y_raw, y_t = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear(dx, dw, db, y_raw, M, N, K)
    capi.linear_tiled(dx, dt, db, y_t, M, N, K)
    got_raw, got_t = to_host(y_raw), to_host(y_t)
    assert np.isfinite(got_raw).all() and np.isfinite(got_t).all()  # every element written
    rng = np.random.default_rng(i)
    rows = np.unique(np.concatenate([[0, N - 1], rng.integers(0, N, size=min(N, 24))]))
    rb = (K // 32) * 34
    w_rows = np.ascontiguousarray(w.reshape(N, rb)[rows]).reshape(-1)
    want = orc.linear(x, w_rows, b[rows] if bias else None, M, rows.size, K)
    bar = 1e-2 if M >= 64 else 1e-5
    assert rel_l2(got_raw[:, rows], want) <= bar, "raw vs oracle"
    assert rel_l2(got_t[:, rows], want) <= bar, "tiled vs oracle"
    assert rel_l2(got_t, got_raw) <= (1e-2 if M >= 64 else 1e-6), "tiled vs raw"
