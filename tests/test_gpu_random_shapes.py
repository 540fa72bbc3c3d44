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
outputs start as NaN).  The same for multi-output Linears and gate/up SwiGLU pairs.
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


def _fused_cases(n=16, seed=1202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.choice([1, 2, 3, 4, 6, 8, 13, 64, 100]))
        KB = int(rng.choice([int(rng.integers(1, 60)), int(rng.integers(60, 140))]))
        Ns = tuple(int(rng.integers(1, 9000)) for _ in range(int(rng.integers(2, 4))))
        out.append((i, M, Ns, 32 * KB))
    # fixed: 512-1024 row groups per weight (the row-range SwiGLU), 4096-element rows
    return out + [(16, 4, (11008, 11008), 4096), (17, 8, (8200, 8200, 1000), 2048)]


FUSED = _fused_cases()


def _silu_mul(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


@pytest.mark.parametrize("i,M,Ns,K", FUSED)
def test_random_fused_shapes(dev, orc, i, M, Ns, K):
    """Multi-output Linear over the random outputs and the SwiGLU pair over the first two
    weights (cut to the first output count): raw and tiled against the oracle on sampled
    rows at the path's bar and against each other."""
    import torch
    note(f"random fused #{i}: M={M} Ns={Ns} K={K}")
    x = S.activations(1000 + i, (M, K))
    ws = [S.q8_0_weight(1100 + 7 * i + j, n, K)[0] for j, n in enumerate(Ns)]
    bs = [S.activations(1200 + 7 * i + j, (n,), tag=S.TAG_BIAS) if j != 1 else None
          for j, n in enumerate(Ns)]
    dx = to_dev(x, dev)
    dws = [to_dev(w, dev) for w in ws]
    dts = []
    for dw, n in zip(dws, Ns):
        t = torch.empty(capi.tiled_bytes(n, K), dtype=torch.uint8, device=dev)
        capi.tile(dw, t, n, K)
        dts.append(t)
    dbs = [to_dev(b, dev) if b is not None else None for b in bs]
    yr = [empty_f32((M, n), dev) for n in Ns]
    yt = [empty_f32((M, n), dev) for n in Ns]
    capi.linear_multi(dx, dws, dbs, yr, list(Ns), M, K)
    capi.linear_multi_tiled(dx, dts, dbs, yt, list(Ns), M, K)
    bar = 1e-2 if M >= 64 else 1e-5
    rng = np.random.default_rng(i)
    for j, n in enumerate(Ns):
        got_r, got_t = to_host(yr[j]), to_host(yt[j])
        assert np.isfinite(got_r).all() and np.isfinite(got_t).all(), j
        rows = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, size=min(n, 16))]))
        w_rows = np.ascontiguousarray(ws[j].reshape(n, -1)[rows]).reshape(-1)
        want = orc.linear(x, w_rows, bs[j][rows] if bs[j] is not None else None, M,
                          rows.size, K)
        assert rel_l2(got_r[:, rows], want) <= bar, ("multi raw", j)
        assert rel_l2(got_t[:, rows], want) <= bar, ("multi tiled", j)
        assert rel_l2(got_t, got_r) <= (1e-2 if M >= 64 else 1e-6), ("multi tiled vs raw", j)
    # SwiGLU over the first two weights, both cut to the first output count's rows
    N = min(Ns[0], Ns[1])
    rb = (K // 32) * 34
    g_raw, u_raw = ws[0][:N * rb], ws[1][:N * rb]
    dg, du = to_dev(g_raw, dev), to_dev(u_raw, dev)
    tg = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
    tu = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
    capi.tile(dg, tg, N, K)
    capi.tile(du, tu, N, K)
    sr, st = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear_swiglu(dx, dg, du, sr, M, N, K)
    capi.linear_swiglu_tiled(dx, tg, tu, st, M, N, K)
    got_r, got_t = to_host(sr), to_host(st)
    assert np.isfinite(got_r).all() and np.isfinite(got_t).all()
    rows = np.unique(np.concatenate([[0, N - 1], rng.integers(0, N, size=min(N, 16))]))
    gr = np.ascontiguousarray(g_raw.reshape(N, rb)[rows]).reshape(-1)
    ur = np.ascontiguousarray(u_raw.reshape(N, rb)[rows]).reshape(-1)
    want = _silu_mul(orc.sgemm_nt(x, gr, M, rows.size, K), orc.sgemm_nt(x, ur, M, rows.size, K))
    assert rel_l2(got_r[:, rows], want) <= bar, "swiglu raw"
    assert rel_l2(got_t[:, rows], want) <= bar, "swiglu tiled"
    assert rel_l2(got_t, got_r) <= (1e-2 if M >= 64 else 1e-6), "swiglu tiled vs raw"


def _matmul_cases(n=14, seed=1203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.choice([1, 2, 5, 8, 9, 17, 40, 63, 64, 90, 200]))
        N = 32 * int(rng.choice([int(rng.integers(1, 20)), int(rng.integers(20, 200))]))
        K = 32 * int(rng.choice([int(rng.integers(1, 10)), int(rng.integers(10, 160))]))
        out.append((i, M, N, K))  # K and N multiples of 32, as the reference requires
    return out


@pytest.mark.parametrize("i,M,N,K", _matmul_cases())
def test_random_matmul_shapes(dev, orc, i, M, N, K):
    """MatMul C = A . B (B [K, N] in blocks along N) over its three kernels (up to 8
    rows of A, 9-63, the bf16 GEMM from 64) on random shapes against the oracle's
    cpu::sgemm restatement (cpu_kernels.cpp:116-130): relative L2 1e-5 below 64 rows,
    1e-2 on the GEMM; repeatable bit for bit."""
    import torch
    note(f"random matmul #{i}: M={M} N={N} K={K}")
    b = S.q8_0_weight(1300 + i, K, N)[0]
    a = S.activations(1400 + i, (M, K))
    da, db = to_dev(a, dev), to_dev(b, dev)
    c1, c2 = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.matmul(da, db, c1, M, N, K)
    capi.matmul(da, db, c2, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    got = to_host(c1)
    assert np.isfinite(got).all()
    assert rel_l2(got, orc.sgemm(a, b, M, N, K)) <= (1e-2 if M >= 64 else 1e-5)
