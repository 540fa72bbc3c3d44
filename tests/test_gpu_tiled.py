"""GPU parity of the Q8_0 16-row tile entry points.

* ``mle_q8_0_tile``: the device repack, byte for byte against the numpy tiler of
  ``helpers.tile_ref`` (itself pinned by a round trip and by explicit loops over
  the layout formula in the CPU tests).
* ``mle_q8_0_linear_tiled`` / ``_swiglu_tiled`` / ``_multi_tiled``: bit for bit
  against the raw entry points wherever both run the MFMA decode or the bf16
  MFMA GEMM (same arithmetic, same accumulation order); where the tiled entry
  point runs its FP32 GEMV (one token, two below vocabulary-sized outputs, up to
  four on short rows: ``tiled_gemv`` below mirrors the C ABI's choice), its
  row-range MFMA decode (``helpers.rows_decode``) or its hybrid MFMA decode
  (``helpers.hybrid_decode``) within relative L2 1e-6 of the raw entry point; and
  always against the CPU oracle
  (reference cpu_kernels.cpp:208-218) at the Linear bars: relative L2 <= 1e-5
  for M < 64 (FP32 GEMV, FP32-exact MFMA decode), <= 1e-2 for M >= 64 (bf16
  GEMM).
"""
import functools

import numpy as np
import pytest

from helpers import (assert_bitexact, empty_f32, hybrid_decode, note, rel_l2, rows_decode,
                     rows_decode_multi,
                     rows_decode_swiglu,
                     tile_ref, to_dev, to_host)
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu


def tol(M):
    return 1e-5 if M < 64 else 1e-2


def tiled_gemv(M, rows, K):
    """The C ABI's choice of the tiled FP32 GEMV (mle::gemv_tiled_wins)."""
    return M == 1 or (M == 2 and rows < 65536) or (M <= 4 and K <= 1024 and rows <= 32768)


def same_or_close(got, want, exact, what):
    """Bit-exact when both sides run the same kernel arithmetic, else equal
    non-finite entries and relative L2 <= 1e-6 over the finite ones."""
    if exact:
        assert_bitexact(got, want, what)
        return
    got, want = np.asarray(got), np.asarray(want)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), what
    nf = ~fin
    assert_bitexact(got[nf], want[nf], what + " (non-finite)")
    assert rel_l2(got[fin], want[fin]) <= 1e-6, what


@functools.lru_cache(maxsize=None)
def weight(seed, rows, cols):
    return S.q8_0_weight(seed, rows, cols)[0]


def tiled_dev(raw_dev, N, K, dev):
    """Device repack of a raw weight already on the device."""
    import torch
    t = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
    capi.tile(raw_dev, t, N, K)
    return t


def silu_mul(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


@pytest.mark.parametrize("N,K", [(1, 32), (17, 96), (100, 4128), (1000, 992), (4096, 11008)])
def test_tile_kernel_matches_reference(dev, N, K):
    note(f"tile N={N} K={K}")
    raw = weight(90 + N, N, K)
    t = tiled_dev(to_dev(raw, dev), N, K, dev)
    got = to_host(t)
    want = tile_ref(raw, N, K)
    assert got.size == want.size
    diff = np.nonzero(got != want)[0]
    assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:5]}"


# (M, N, K, bias): MFMA decode cases (raw path 3: M >= 2 with K > 1024 or M > 4),
# the decode in 16-token chunks, and GEMM cases; N not a multiple of 16 and odd
# K/32 (a zero block pads the last pair) included.
CASES = [(2, 4096, 4096, False), (4, 11008, 4096, True), (5, 1000, 4128, True),
         (8, 4096, 11008, False), (8, 12288, 4096, False), (13, 777, 2048, True),
         (16, 96, 992, False), (17, 96, 992, True), (33, 200, 512, False),
         (63, 64, 1024, True), (64, 192, 256, False), (100, 1000, 4128, True),
         (129, 160, 992, False), (512, 4096, 4096, False)]


@pytest.mark.parametrize("M,N,K,has_bias", CASES)
def test_linear_tiled_matches_raw_and_oracle(dev, orc, M, N, K, has_bias):
    note(f"linear_tiled M={M} N={N} K={K} bias={has_bias}")
    raw = weight(N + 7, N, K)
    x = S.activations(K + M, (M, K))
    bias = S.activations(N, (N,), tag=S.TAG_BIAS) if has_bias else None
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    db = to_dev(bias, dev) if has_bias else None
    dt = tiled_dev(dw, N, K, dev)
    y_raw, y_t = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear(dx, dw, db, y_raw, M, N, K)
    capi.linear_tiled(dx, dt, db, y_t, M, N, K)
    got = to_host(y_t)
    # bit for bit where both run the split-K MFMA decode or the GEMM (the tiled GEMV,
    # the row-range and the hybrid decode group the K sum differently)
    exact = not tiled_gemv(M, N, K) and not rows_decode(M, N, K) and not hybrid_decode(M, N, K)
    same_or_close(got, to_host(y_raw), exact, "tiled vs raw")
    if M * N * K <= 64 * 1024 * 1024:
        assert rel_l2(got, orc.linear(x, raw, bias, M, N, K)) <= tol(M)
    else:  # sampled rows against the oracle
        rows = np.array([0, M // 2, M - 1])
        want = orc.linear(x[rows], raw, bias, rows.size, N, K)
        assert rel_l2(got[rows], want) <= tol(M)


@pytest.mark.parametrize("M,N,K,has_bias", [
    (1, 4096, 4096, False), (1, 11008, 4096, True), (1, 4096, 11008, False),
    (1, 1152, 896, True), (1, 151936, 896, False), (1, 100, 4128, True), (1, 1000, 992, False),
    (1, 17, 32, True), (2, 4096, 4096, False), (2, 896, 4864, True), (3, 4864, 896, False),
    (4, 300, 512, True), (4, 1152, 896, False)])
def test_linear_tiled_gemv(dev, orc, M, N, K, has_bias):
    """The tiled FP32 GEMV (M == 1, M == 2, short rows): against the oracle, the
    raw entry point, and itself (deterministic)."""
    import torch
    assert tiled_gemv(M, N, K)
    note(f"linear_tiled gemv M={M} N={N} K={K} bias={has_bias}")
    raw = weight(N + 3, N, K)
    x = S.activations(K + 11 * M, (M, K))
    bias = S.activations(N + 1, (N,), tag=S.TAG_BIAS) if has_bias else None
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    db = to_dev(bias, dev) if has_bias else None
    dt = tiled_dev(dw, N, K, dev)
    y_t, y_t2, y_raw = (empty_f32((M, N), dev) for _ in range(3))
    capi.linear_tiled(dx, dt, db, y_t, M, N, K)
    capi.linear_tiled(dx, dt, db, y_t2, M, N, K)
    capi.linear(dx, dw, db, y_raw, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_t2)
    got = to_host(y_t)
    same_or_close(got, to_host(y_raw), False, "tiled gemv vs raw")
    assert rel_l2(got, orc.linear(x, raw, bias, M, N, K)) <= tol(M)


def test_linear_tiled_special_values(dev):
    """Inf / NaN activations propagate exactly as on the raw path."""
    M, N, K = 8, 256, 2048
    raw = weight(41, N, K)
    x = S.activations(42, (M, K))
    x[1, 5] = np.inf
    x[2, 100] = -np.inf
    x[3, 7] = np.nan
    x[4, :] = 0.0
    x[5, 3] = 3.0e38
    note("linear_tiled special values")
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    y_raw, y_t = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear(dx, dw, None, y_raw, M, N, K)
    capi.linear_tiled(dx, dt, None, y_t, M, N, K)
    assert_bitexact(to_host(y_t), to_host(y_raw), "special values")
    # the GEMM (M >= 64) on rows carrying the same values: bit for bit
    M2 = 70
    x2 = np.concatenate([x, S.activations(43, (M2 - M, K))])
    dx2 = to_dev(x2, dev)
    y2r, y2t = empty_f32((M2, N), dev), empty_f32((M2, N), dev)
    capi.linear(dx2, dw, None, y2r, M2, N, K)
    capi.linear_tiled(dx2, dt, None, y2t, M2, N, K)
    assert_bitexact(to_host(y2t), to_host(y2r), "special values gemm")
    # the tiled GEMV (one token) on the same rows: non-finite entries as the raw
    # GEMV gives them
    for row in (1, 3, 4):
        y1r, y1t = empty_f32((1, N), dev), empty_f32((1, N), dev)
        capi.linear(dx[row:row + 1], dw, None, y1r, 1, N, K)
        capi.linear_tiled(dx[row:row + 1], dt, None, y1t, 1, N, K)
        same_or_close(to_host(y1t), to_host(y1r), False, f"special values gemv row {row}")


@pytest.mark.parametrize("M,N,K", [(1, 300, 512), (2, 1000, 4096), (8, 11008, 4096),
                                   (17, 96, 992), (40, 130, 64), (64, 192, 256),
                                   (100, 320, 1024), (512, 11008, 4096)])
def test_swiglu_tiled(dev, orc, M, N, K):
    import torch
    note(f"swiglu_tiled M={M} N={N} K={K}")
    wg, wu = weight(60 + N, N, K), weight(61 + N, N, K)
    x = S.activations(62 + K, (M, K))
    dx, dwg, dwu = to_dev(x, dev), to_dev(wg, dev), to_dev(wu, dev)
    tg, tu = tiled_dev(dwg, N, K, dev), tiled_dev(dwu, N, K, dev)
    y_raw, y_t = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear_swiglu(dx, dwg, dwu, y_raw, M, N, K)
    capi.linear_swiglu_tiled(dx, tg, tu, y_t, M, N, K)
    got = to_host(y_t)
    # raw SwiGLU runs its GEMV for M == 1 only; tiled, its GEMV as tiled_gemv says,
    # and the row-range decode where rows_decode_swiglu says
    exact = M > 1 and not tiled_gemv(M, N, K) and not rows_decode_swiglu(M, N, K)
    same_or_close(got, to_host(y_raw), exact, "swiglu tiled vs raw")
    rows = np.array(sorted({0, M // 2, M - 1}))
    want = silu_mul(orc.linear(x[rows], wg, None, rows.size, N, K),
                    orc.linear(x[rows], wu, None, rows.size, N, K))
    assert rel_l2(got[rows], want) <= tol(M)
    y2 = empty_f32((M, N), dev)
    capi.linear_swiglu_tiled(dx, tg, tu, y2, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y_t, y2)


@pytest.mark.parametrize("M", [1, 2, 5, 16, 40, 70])
def test_multi_tiled(dev, orc, M):
    import torch
    K = 512
    Ns = (160, 96, 40)
    ws = [weight(70 + i, n, K) for i, n in enumerate(Ns)]
    biases = [S.activations(80, (Ns[0],), tag=S.TAG_BIAS), None,
              S.activations(82, (Ns[2],), tag=S.TAG_BIAS)]
    x = S.activations(83, (M, K))
    note(f"multi_tiled M={M} Ns={Ns}")
    dx = to_dev(x, dev)
    dws = [to_dev(w, dev) for w in ws]
    dts = [tiled_dev(w, n, K, dev) for w, n in zip(dws, Ns)]
    dbs = [to_dev(b, dev) if b is not None else None for b in biases]
    ys = [empty_f32((M, n), dev) for n in Ns]
    capi.linear_multi_tiled(dx, dts, dbs, ys, Ns, M, K)
    torch.cuda.synchronize()
    for i, n in enumerate(Ns):
        got = to_host(ys[i])
        assert rel_l2(got, orc.linear(x, ws[i], biases[i], M, n, K)) <= tol(M), i
        if M < 64:  # one output of the fused launch against the single tiled Linear
            single = empty_f32((M, n), dev)
            capi.linear_tiled(dx, dts[i], dbs[i], single, M, n, K)
            # same MFMA decode K slices: same bits; the GEMV splits K by launch shape
            exact = not tiled_gemv(M, sum(Ns), K) and not tiled_gemv(M, n, K)
            same_or_close(to_host(ys[i]), to_host(single), exact, f"multi {i}")
    if M >= 64:  # the fused GEMM: raw and tiled weights give the same bits
        yr = [empty_f32((M, n), dev) for n in Ns]
        capi.linear_multi(dx, dws, dbs, yr, Ns, M, K)
        for i in range(3):
            assert_bitexact(to_host(ys[i]), to_host(yr[i]), f"multi {i}")


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_llama_decode_set_tiled(dev, M):
    """The four Llama-7B projection shapes of the decode benchmark, tiled against
    raw on the fused qkv, the fused gate/up and o_proj / down: bit for bit on the
    split-K MFMA decode (M = 4, 8), within 1e-6 on the tiled GEMV (M = 1, 2) and on
    the row-range decode (o_proj at M = 4, the fused q/k/v and gate/up at M = 4 and
    8)."""
    import torch
    K, H, F = 4096, 4096, 11008
    note(f"llama decode set tiled M={M}")
    x = to_dev(S.activations(7, (M, K)), dev)
    xf = to_dev(S.activations(8, (M, F)), dev)
    raw = {n: to_dev(weight(s, r, c), dev) for n, s, r, c in
           [("q", 1, H, K), ("k", 2, H, K), ("v", 3, H, K), ("o", 4, H, K),
            ("gate", 5, F, K), ("up", 6, F, K), ("down", 9, H, F)]}
    shape = {"q": (H, K), "k": (H, K), "v": (H, K), "o": (H, K), "gate": (F, K),
             "up": (F, K), "down": (H, F)}
    til = {n: tiled_dev(w, *shape[n], dev) for n, w in raw.items()}
    ys_r = [empty_f32((M, H), dev) for _ in range(3)]
    ys_t = [empty_f32((M, H), dev) for _ in range(3)]
    capi.linear_multi(x, [raw["q"], raw["k"], raw["v"]], None, ys_r, (H, H, H), M, K)
    capi.linear_multi_tiled(x, [til["q"], til["k"], til["v"]], None, ys_t, (H, H, H), M, K)
    g_r, g_t = empty_f32((M, F), dev), empty_f32((M, F), dev)
    capi.linear_swiglu(x, raw["gate"], raw["up"], g_r, M, F, K)
    capi.linear_swiglu_tiled(x, til["gate"], til["up"], g_t, M, F, K)
    o_r, o_t = empty_f32((M, H), dev), empty_f32((M, H), dev)
    capi.linear(x, raw["o"], None, o_r, M, H, K)
    capi.linear_tiled(x, til["o"], None, o_t, M, H, K)
    d_r, d_t = empty_f32((M, H), dev), empty_f32((M, H), dev)
    capi.linear(xf, raw["down"], None, d_r, M, H, F)
    capi.linear_tiled(xf, til["down"], None, d_t, M, H, F)
    torch.cuda.synchronize()
    for a, b, what in [(ys_r[0], ys_t[0], "q"), (ys_r[1], ys_t[1], "k"),
                       (ys_r[2], ys_t[2], "v"), (g_r, g_t, "gate/up"), (o_r, o_t, "o"),
                       (d_r, d_t, "down")]:
        # the row-range decode on tiled weights: o_proj at M = 4, q/k/v and the
        # gate/up SwiGLU at M = 4 and 8; the hybrid decode: down at M = 4 and 8
        other = (rows_decode(M, H, K) if what == "o" else
                 rows_decode_multi(M, (H, H, H), K) if what in "qkv" else
                 rows_decode_swiglu(M, F, K) if what == "gate/up" else
                 hybrid_decode(M, H, F))
        exact = M > 2 and not other
        same_or_close(to_host(b), to_host(a), exact, what)
