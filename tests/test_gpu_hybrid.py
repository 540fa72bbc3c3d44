"""GPU parity of the hybrid MFMA decode: tiled and raw weights, 3-8 tokens, each
workgroup owning a few 16-row groups and one short split of K (mle::decode_mfma_pick
takes it for rows of 8192+ elements over at most 256 groups, the Llama down
projection).

Checked against the CPU oracle (reference cpu_kernels.cpp:208-218) at the decode
bar, relative L2 <= 1e-5; against the split-K MFMA decode on the raw bytes within
relative L2 1e-6 with equal non-finite entries (both sum the same exact block
products, grouped differently over K); the same launch shape on the raw bytes bit
for bit (raw lanes load whole blocks and transpose them into the same A fragments);
repeatable bit for bit.  Every launch shape
of the kernel (mle_q8_0_linear_tiled_ex, t3 = 1..4: 4 / 8 / 16 groups per
workgroup, 1-4 waves per group, 22-44-block splits, 1-3 load chunks in flight) runs
on ragged shapes: N not a multiple of 16 and fewer groups than a workgroup holds,
K with an odd number of blocks and a last split shorter than the others, K in one
split (no hand-off), fp32 and bf16 bias, special activations, and a multi-output
launch whose segment boundary falls inside a workgroup.
"""
import functools

import numpy as np
import pytest

from helpers import (assert_bitexact, empty_f32, hybrid_decode, note, rel_l2, to_dev,
                     to_host)
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-5
SHAPES = (1, 2, 3, 4)


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


def check_against_oracle(orc, x, raw, b32, got, M, N, K):
    rows = np.array(sorted({0, 1, N // 2, max(N - 17, 0), N - 1}))
    w_rows = np.ascontiguousarray(raw.reshape(N, -1)[rows]).reshape(-1)
    want = orc.linear(x, w_rows, b32[rows] if b32 is not None else None, M, rows.size, K)
    assert rel_l2(got[:, rows], want) <= DECODE_TOL
    if M * N * K <= 8 * 2048 * 11008:
        assert rel_l2(got, orc.linear(x, raw, b32, M, N, K)) <= DECODE_TOL


def test_picker_takes_hybrid_for_llama_down():
    assert hybrid_decode(4, 4096, 11008) and hybrid_decode(8, 4096, 11008)
    assert not hybrid_decode(8, 4096, 4096) and not hybrid_decode(5, 4096, 11008)
    assert not hybrid_decode(1, 4096, 11008) and not hybrid_decode(8, 11008, 11008)


# (M, N, K, bias): the Llama down shape; N past a 16-row group and fewer groups
# than a workgroup holds; K = 343 blocks (odd: a half pair) and 346 blocks (a last
# split of 38 blocks); K in one split (no hand-off).
CASES = [(8, 4096, 11008, None), (4, 4096, 11008, "f32"), (3, 4000, 10976, "bf16"),
         (7, 200, 11072, None), (6, 1040, 8192, "f32"), (4, 48, 1024, None),
         (8, 2064, 640, "bf16")]


@pytest.mark.parametrize("hyb", SHAPES)
@pytest.mark.parametrize("M,N,K,bias", CASES)
def test_hybrid_matches_oracle_and_split_k(dev, orc, hyb, M, N, K, bias):
    import torch
    note(f"hybrid decode shape {hyb} M={M} N={N} K={K} bias={bias}")
    raw = weight(N + K, N, K)
    x = S.activations(K + 3 * M, (M, K))
    b32 = S.activations(N + 9, (N,), tag=S.TAG_BIAS) if bias else None
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    mt = 4 if M <= 4 else 8
    y, y2, y_raw = (empty_f32((M, N), dev) for _ in range(3))
    if bias == "bf16":
        b16 = torch.from_numpy(b32).to(dev).to(torch.bfloat16)
        b32 = b16.float().cpu().numpy()  # the widened bias the oracle adds
        db = b16.float()  # the forced-shape hook takes an fp32 bias: the widened values
    else:
        db = to_dev(b32, dev) if bias else None
    capi.linear_ex(dx, dt, db, y, M, N, K, path=3, mt=mt, hyb=hyb, tiled=True)
    capi.linear_ex(dx, dt, db, y2, M, N, K, path=3, mt=mt, hyb=hyb, tiled=True)
    capi.linear_ex(dx, dw, db, y_raw, M, N, K, path=3, mt=mt, waves=4, kslice=16)
    y_rh = empty_f32((M, N), dev)
    capi.linear_ex(dx, dw, db, y_rh, M, N, K, path=3, mt=mt, hyb=hyb)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)  # deterministic
    got = to_host(y)
    close_to_raw(got, to_host(y_raw), "hybrid vs split-K")
    assert_bitexact(to_host(y_rh), got, "raw vs tiled hybrid")
    check_against_oracle(orc, x, raw, b32, got, M, N, K)


@pytest.mark.parametrize("M,N,K,bias", [(8, 4096, 11008, "f32"), (4, 4096, 11008, "bf16"),
                                        (3, 3000, 9216, None), (6, 256, 8192, "f32")])
def test_hybrid_picked_by_tiled_linear(dev, orc, M, N, K, bias):
    """mle_q8_0_linear_tiled (and the bf16-bias entry point) on the shapes the
    picker gives the hybrid kernel: equal to the forced launch shape 1 bit for bit,
    and so is the raw entry point (the same kernel on the raw bytes); within 1e-6 of
    the split-K raw launch, at the decode bar against the oracle, and with its split-K
    workspace (partials and one counter per workgroup column) reported by the C ABI
    for either layout."""
    import torch
    assert hybrid_decode(M, N, K)
    note(f"hybrid picked M={M} N={N} K={K} bias={bias}")
    raw = weight(N + 2 * K, N, K)
    x = S.activations(K + 11 * M, (M, K))
    b32 = S.activations(N + 4, (N,), tag=S.TAG_BIAS) if bias else None
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    y, y_forced, y_raw = (empty_f32((M, N), dev) for _ in range(3))
    if bias == "bf16":
        b16 = torch.from_numpy(b32).to(dev).to(torch.bfloat16)
        b32 = b16.float().cpu().numpy()
        capi.linear_bias_bf16(dx, dt, b16, y, M, N, K, tiled=True)
        db = b16.float()
    else:
        db = to_dev(b32, dev) if bias else None
        capi.linear_tiled(dx, dt, db, y, M, N, K)
    capi.linear_ex(dx, dt, db, y_forced, M, N, K, path=3, mt=4 if M <= 4 else 8, hyb=1,
                   tiled=True)
    capi.linear_ex(dx, dw, db, y_raw, M, N, K, path=3, mt=4 if M <= 4 else 8, waves=4,
                   kslice=16)
    y_auto_raw = empty_f32((M, N), dev)
    capi.linear(dx, dw, db, y_auto_raw, M, N, K)
    torch.cuda.synchronize()
    got = to_host(y)
    assert_bitexact(got, to_host(y_forced), "picked vs forced shape 1")
    assert_bitexact(to_host(y_auto_raw), got, "raw entry point vs tiled")
    close_to_raw(got, to_host(y_raw), "hybrid vs split-K")
    check_against_oracle(orc, x, raw, b32, got, M, N, K)
    G = (N + 15) // 16
    tiles, splits, mt = (G + 3) // 4, (K // 32 + 43) // 44, 4 if M <= 4 else 8
    for tiled in (True, False):
        b, c = capi.workspace_size(capi.OP_LINEAR, M, [N], K, tiled)
        if splits > 1:
            assert b >= tiles * splits * 4 * 16 * mt * 4 and c >= tiles * 32
        else:
            assert (b, c) == (0, 0)


@pytest.mark.parametrize("hyb", SHAPES)
def test_hybrid_special_values(dev, hyb):
    """Inf, NaN, zero rows and large finite activations: the same non-finite
    entries as the split-K kernel on raw weights, the finite ones within 1e-6."""
    M, N, K = 8, 1024, 11008
    raw = weight(93, N, K)
    x = S.activations(94, (M, K))
    x[1, 5] = np.inf
    x[2, 10000] = -np.inf
    x[3, 7] = np.nan
    x[4, :] = 0.0
    x[5, 3] = 1.0e30
    x[6, 1500] = np.inf
    x[6, 9000] = -np.inf
    note(f"hybrid special values shape {hyb}")
    dx, dw = to_dev(x, dev), to_dev(raw, dev)
    dt = tiled_dev(dw, N, K, dev)
    y_raw, y, y_rh = (empty_f32((M, N), dev) for _ in range(3))
    capi.linear_ex(dx, dw, None, y_raw, M, N, K, path=3, mt=8, waves=4, kslice=16)
    capi.linear_ex(dx, dt, None, y, M, N, K, path=3, mt=8, hyb=hyb, tiled=True)
    capi.linear_ex(dx, dw, None, y_rh, M, N, K, path=3, mt=8, hyb=hyb)
    got, want = to_host(y), to_host(y_raw)
    assert np.isnan(got[3]).all()
    assert (got[4] == 0).all()
    assert not np.isfinite(got[[1, 2, 6]]).any()
    close_to_raw(got, want, "special values")
    assert_bitexact(to_host(y_rh), got, "raw vs tiled hybrid, special values")


@pytest.mark.parametrize("M,Ns,K", [(8, (2000, 2096), 11008), (4, (1000, 24, 3056), 8192)])
def test_hybrid_multi_output(dev, orc, M, Ns, K):
    """A multi-output Linear on the hybrid decode: 125 + 131 groups (the segment
    boundary inside a 4-group workgroup) and three outputs of 63 + 2 + 191 groups.
    Each output against the oracle on sampled rows, against its single tiled Linear
    within 1e-6, with its own bias; repeatable bit for bit; the raw multi-output launch
    (the same kernel on the raw bytes) gives the same bits."""
    import torch
    G = sum((n + 15) // 16 for n in Ns)
    assert hybrid_decode(M, 16 * G, K)
    note(f"hybrid multi M={M} Ns={Ns} K={K}")
    raws = [weight(500 + 7 * i + n, n, K) for i, n in enumerate(Ns)]
    x = S.activations(501 + M, (M, K))
    biases = [S.activations(502 + i, (n,), tag=S.TAG_BIAS) if i != 1 else None
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
    for i, n in enumerate(Ns):
        assert torch.equal(ys[i], ys2[i]), i
        assert torch.equal(ys[i], yr[i]), ("raw vs tiled", i)
        got = to_host(ys[i])
        single = empty_f32((M, n), dev)
        capi.linear_tiled(dx, dts[i], dbs[i], single, M, n, K)
        close_to_raw(got, to_host(single), f"multi {i} vs single")
        rows = np.array(sorted({0, n // 3, n - 1}))
        w_rows = np.ascontiguousarray(raws[i].reshape(n, -1)[rows]).reshape(-1)
        b = biases[i][rows] if biases[i] is not None else None
        assert rel_l2(got[:, rows], orc.linear(x, w_rows, b, M, rows.size, K)) <= DECODE_TOL, i


def test_forced_hybrid_shape_rejected_outside_its_range(dev):
    """The tuning hook accepts hybrid shapes 1-4 only."""
    M, N, K = 4, 64, 1024
    dx = to_dev(S.activations(1, (M, K)), dev)
    dt = tiled_dev(to_dev(weight(2, N, K), dev), N, K, dev)
    y = empty_f32((M, N), dev)
    with pytest.raises(capi.Q8_0Error):
        capi.linear_ex(dx, dt, None, y, M, N, K, path=3, mt=4, hyb=5, tiled=True)
