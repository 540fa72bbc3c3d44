"""GPU parity of the row-range MFMA decode: tiled weights, K 2048-4096 in steps of
64, 3-8 tokens on 512-1024 16-row groups or 3-4 tokens on 240-256 groups (the
launches for which mle::decode_mfma_pick sets DecodeMfmaConfig::rows).  Each workgroup owns whole
16-row groups and all of K, so there is no split-K hand-off and no workspace.

Checked against the CPU oracle (reference cpu_kernels.cpp:208-218) at the decode
bar, relative L2 <= 1e-5; against the split-K MFMA decode on raw weights within
relative L2 1e-6 with equal non-finite entries (both sum the same exact block
products, grouped differently over K); against the raw entry point bit for bit where
it runs the row-range kernel too (3-4 tokens on 512-1024 groups: raw lanes load
whole blocks and transpose them into the same A fragments), else within 1e-6;
repeatable bit for bit;
and with a zero workspace need reported by the C ABI.  Cases cover 1 to 4
groups per workgroup, one to four K phases (single and double buffered), N not
a multiple of 16 (a partial last group), an odd number of block pairs, fp32 and bf16
bias, and Inf / NaN / large activations.
"""
import functools

import numpy as np
import pytest

from helpers import (assert_bitexact, empty_f32, note, rel_l2, rows_decode, rows_decode_multi,
                     rows_decode_raw, rows_decode_swiglu,
                     to_dev, to_host)
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-5


@functools.lru_cache(maxsize=None)
def weight(seed, rows, cols):
    return S.q8_0_weight(seed, rows, cols)[0]


def tiled_dev(raw_dev, N, K, dev):
    import torch
    t = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
    capi.tile(raw_dev, t, N, K)
    return t


def close_to_raw(got, raw, what):
    fin = np.isfinite(raw)
    assert np.array_equal(np.isfinite(got), fin), what
    assert_bitexact(got[~fin], raw[~fin], what + " (non-finite)")
    assert rel_l2(got[fin], raw[fin]) <= 1e-6, what


# (M, N, K, bias): groups per workgroup 1 (G = 240-256, 16 waves on the group),
# 2 (G = 512), 3 (G = 513, 688, 768) and 4 (G = 1024); MT 4 (K in one phase) and
# MT 8 (32-block phases in two buffers: 2, 3 and 4 phases; K = 2112 leaves the
# last phase with two blocks, one pair).
CASES = [(3, 8192, 2048, None), (4, 11008, 4096, "f32"), (4, 16384, 4096, None),
         (4, 8200, 2112, "bf16"), (4, 4096, 4096, None), (3, 3900, 3072, "f32"),
         (4, 3840, 2048, None), (6, 8200, 2112, None), (7, 12288, 4096, "bf16"),
         (8, 11008, 4096, None), (8, 16384, 3072, "f32"), (8, 8192, 4096, None),
         (8, 8192, 2048, None)]


@pytest.mark.parametrize("M,N,K,bias", CASES)
def test_rows_decode_matches_oracle_and_split_k(dev, orc, M, N, K, bias):
    import torch
    assert rows_decode(M, N, K)
    note(f"rows decode M={M} N={N} K={K} bias={bias}")
    raw = weight(N + K, N, K)
    x = S.activations(K + 5 * M, (M, K))
    b32 = S.activations(N + 2, (N,), tag=S.TAG_BIAS) if bias else None
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    y_t, y_t2, y_raw, y_sk = (empty_f32((M, N), dev) for _ in range(4))
    if bias == "bf16":
        b16 = torch.from_numpy(b32).to(dev).to(torch.bfloat16)
        b32 = b16.float().cpu().numpy()  # the widened bias the oracle adds
        capi.linear_bias_bf16(dx, dt, b16, y_t, M, N, K, tiled=True)
        capi.linear_bias_bf16(dx, dt, b16, y_t2, M, N, K, tiled=True)
        capi.linear_bias_bf16(dx, dw, b16, y_raw, M, N, K)
    else:
        db = to_dev(b32, dev) if bias else None
        capi.linear_tiled(dx, dt, db, y_t, M, N, K)
        capi.linear_tiled(dx, dt, db, y_t2, M, N, K)
        capi.linear(dx, dw, db, y_raw, M, N, K)
    # the split-K kernel on raw weights (forced launch shape), widened bias
    capi.linear_ex(dx, dw, to_dev(b32, dev) if bias else None, y_sk, M, N, K, path=3,
                   mt=4 if M <= 4 else 8, waves=8, kslice=16)
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_t2)  # deterministic
    got = to_host(y_t)
    close_to_raw(got, to_host(y_sk), "rows vs split-K")
    if rows_decode_raw(M, N, K):
        assert_bitexact(got, to_host(y_raw), "tiled vs raw row-range")
    else:
        close_to_raw(got, to_host(y_raw), "tiled rows vs raw")
    rows = np.array(sorted({0, 1, N // 2, N - 17, N - 1}))
    w_rows = np.ascontiguousarray(raw.reshape(N, -1)[rows]).reshape(-1)
    want = orc.linear(x, w_rows, b32[rows] if bias else None, M, rows.size, K)
    assert rel_l2(got[:, rows], want) <= DECODE_TOL
    if M * N * K <= 8 * 8192 * 2048:  # the whole output on the smaller shapes
        assert rel_l2(got, orc.linear(x, raw, b32, M, N, K)) <= DECODE_TOL
    assert capi.workspace_size(capi.OP_LINEAR, M, [N], K, True) == (0, 0)


def test_rows_decode_special_values(dev):
    """Inf, NaN, zero rows and large finite activations: the same non-finite
    entries as the split-K kernel on raw weights, the finite ones within 1e-6."""
    M, N, K = 8, 8192, 2048
    assert rows_decode(M, N, K)
    raw = weight(91, N, K)
    x = S.activations(92, (M, K))
    x[1, 5] = np.inf
    x[2, 100] = -np.inf
    x[3, 7] = np.nan
    x[4, :] = 0.0
    x[5, 3] = 1.0e30
    x[6, 1500] = np.inf
    x[6, 1501] = -np.inf
    note("rows decode special values")
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    y_raw, y_t = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear(dx, dw, None, y_raw, M, N, K)
    capi.linear_tiled(dx, dt, None, y_t, M, N, K)
    got, want = to_host(y_t), to_host(y_raw)
    assert np.isnan(got[3]).all()
    assert (got[4] == 0).all()
    assert not np.isfinite(got[[1, 2, 6]]).any()
    close_to_raw(got, want, "special values")


def test_rows_decode_raw_special_values(dev):
    """Raw weights at 4 tokens on 512 groups (the raw entry point's row-range
    decode): Inf, NaN and large activations give the tiled launch's bits, including
    the non-finite entries, and the split-K kernel's within 1e-6."""
    import torch
    M, N, K = 4, 8192, 2048
    assert rows_decode_raw(M, N, K)
    raw = weight(93, N, K)
    x = S.activations(94, (M, K))
    x[0, 3] = 1.0e30
    x[1, 5] = np.inf
    x[2, 100] = -np.inf
    x[3, 7] = np.nan
    note("raw rows decode special values")
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    y_raw, y_t, y_sk = (empty_f32((M, N), dev) for _ in range(3))
    capi.linear(dx, dw, None, y_raw, M, N, K)
    capi.linear_tiled(dx, dt, None, y_t, M, N, K)
    capi.linear_ex(dx, dw, None, y_sk, M, N, K, path=3, mt=4, waves=8, kslice=16)
    torch.cuda.synchronize()
    got = to_host(y_raw)
    assert np.isnan(got[3]).all()
    assert not np.isfinite(got[[1, 2]]).any()
    assert_bitexact(got, to_host(y_t), "raw vs tiled row-range")
    close_to_raw(got, to_host(y_sk), "raw row-range vs split-K")
    assert capi.workspace_size(capi.OP_LINEAR, M, [N], K, False) == (0, 0)


@pytest.mark.parametrize("M,Ns,K", [(4, (4096, 4096, 4096), 4096), (8, (4096, 4096, 4096), 4096),
                                    (3, (4000, 4000, 4100), 2048), (7, (8192, 192), 3072),
                                    (4, (3000, 900), 2112)])
def test_rows_decode_multi_output(dev, orc, M, Ns, K):
    """The multi-output Linear (q/k/v) on the row-range decode: segment boundaries
    inside workgroups (250 + 250 + 257 groups over 3-group workgroups), two outputs,
    and 240 groups in one-group workgroups.  Each output against the oracle (sampled
    rows on the larger shapes), against the single tiled Linear within 1e-6, with
    its own bias; repeatable bit for bit; no workspace; the raw multi-output launch
    gives the same bits where it takes the row-range kernel too (3-4 tokens), else
    within 1e-6."""
    import torch
    assert rows_decode_multi(M, Ns, K)
    note(f"rows decode multi M={M} Ns={Ns} K={K}")
    raws = [weight(300 + 7 * i + n, n, K) for i, n in enumerate(Ns)]
    x = S.activations(301 + M, (M, K))
    biases = [S.activations(302 + i, (n,), tag=S.TAG_BIAS) if i != 1 else None
              for i, n in enumerate(Ns)]
    dx = to_dev(x, dev)
    dts = [tiled_dev(to_dev(w, dev), n, K, dev) for w, n in zip(raws, Ns)]
    dbs = [to_dev(b, dev) if b is not None else None for b in biases]
    ys = [empty_f32((M, n), dev) for n in Ns]
    ys2 = [empty_f32((M, n), dev) for n in Ns]
    capi.linear_multi_tiled(dx, dts, dbs, ys, Ns, M, K)
    capi.linear_multi_tiled(dx, dts, dbs, ys2, Ns, M, K)
    yr = [empty_f32((M, n), dev) for n in Ns]
    capi.linear_multi(dx, [to_dev(w, dev) for w in raws], dbs, yr, Ns, M, K)
    torch.cuda.synchronize()
    raw_rows = rows_decode_raw(M, 16 * sum((n + 15) // 16 for n in Ns), K)
    for i, n in enumerate(Ns):
        assert torch.equal(ys[i], ys2[i]), i
        got = to_host(ys[i])
        if raw_rows:
            assert_bitexact(got, to_host(yr[i]), f"multi {i} tiled vs raw")
        else:
            close_to_raw(got, to_host(yr[i]), f"multi {i} tiled vs raw")
        single = empty_f32((M, n), dev)
        capi.linear_tiled(dx, dts[i], dbs[i], single, M, n, K)
        close_to_raw(got, to_host(single), f"multi {i} vs single")
        rows = np.array(sorted({0, n // 3, n - 1}))
        w_rows = np.ascontiguousarray(raws[i].reshape(n, -1)[rows]).reshape(-1)
        b = biases[i][rows] if biases[i] is not None else None
        assert rel_l2(got[:, rows], orc.linear(x, w_rows, b, M, rows.size, K)) <= DECODE_TOL, i
    assert capi.workspace_size(capi.OP_LINEAR_MULTI, M, list(Ns), K, True) == (0, 0)


def silu_mul(g, u):
    """silu(g) * u in the reference's operation order (cpu_kernels.cpp:848-858), fp32."""
    g = np.asarray(g, np.float32)
    return ((g / (np.float32(1.0) + np.exp(-g))) * u).astype(np.float32)


# (M, N, K): gate/up pairs per workgroup 2 (G = 512), 3 (G = 513, 688) and 4
# (G = 1024); MT 4 (K in one phase) and MT 8 (2-4 phases of 32 blocks).
SWIGLU_CASES = [(4, 11008, 4096), (3, 8192, 2048), (4, 8200, 2112), (8, 11008, 4096),
                (6, 16384, 3072), (7, 8200, 2112), (8, 8192, 2048)]


@pytest.mark.parametrize("M,N,K", SWIGLU_CASES)
def test_rows_decode_swiglu(dev, orc, M, N, K):
    """The fused gate/up SwiGLU launch on the row-range decode (gate and up groups of
    the same rows in one workgroup, silu(gate) * up in its epilogue), on tiled and on
    raw weights: against the oracle at the decode bar on sampled rows (each projection
    by the reference's sgemm_nt, then its silu * up order), raw equal to tiled bit for
    bit (whole raw blocks per lane, transposed into the tiled layout's fragments, the
    same K order), repeatable bit for bit, and with no workspace on either layout."""
    import torch
    assert rows_decode_swiglu(M, N, K)
    note(f"rows decode swiglu M={M} N={N} K={K}")
    wg, wu = weight(N + K + 1, N, K), weight(N + K + 2, N, K)
    x = S.activations(K + 7 * M, (M, K))
    dx, dwg, dwu = to_dev(x, dev), to_dev(wg, dev), to_dev(wu, dev)
    tg, tu = tiled_dev(dwg, N, K, dev), tiled_dev(dwu, N, K, dev)
    y_t, y_t2, y_raw = (empty_f32((M, N), dev) for _ in range(3))
    capi.linear_swiglu_tiled(dx, tg, tu, y_t, M, N, K)
    capi.linear_swiglu_tiled(dx, tg, tu, y_t2, M, N, K)
    capi.linear_swiglu(dx, dwg, dwu, y_raw, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_t2)  # deterministic
    got = to_host(y_t)
    assert_bitexact(to_host(y_raw), got, "swiglu rows raw vs tiled")
    rows = np.array(sorted({0, 1, N // 2, N - 17, N - 1}))
    pick = lambda w: np.ascontiguousarray(w.reshape(N, -1)[rows]).reshape(-1)
    want = silu_mul(orc.linear(x, pick(wg), None, M, rows.size, K),
                    orc.linear(x, pick(wu), None, M, rows.size, K))
    assert rel_l2(got[:, rows], want) <= DECODE_TOL
    for tiled in (True, False):
        assert capi.workspace_size(capi.OP_LINEAR_SWIGLU, M, [N, N], K, tiled) == (0, 0)
