"""GPU parity on a weight past 4 GiB: 64-bit addressing on every Linear path and the
Embedding.

A raw Q8_0 weight of 1 000 003 rows x 4096 (4.35 GB, ragged last 16-row group) and its
16-row tiled copy are made on the device.  Blocks near the end of the weight sit past
byte 2^32, where a 32-bit offset would wrap.  The Linear runs at 1, 4, 8 and 64 tokens,
which covers the FP32 GEMV, the tiled GEMV, the split-K MFMA decode (both layouts) and
the bf16 MFMA GEMM.  Outputs start as NaN and every element must be written.  Sampled
rows, including the last ones, are checked against the CPU oracle (reference
cpu_kernels.cpp:208-218) at the path's bar: relative L2 1e-5 below 64 tokens, 1e-2 on
the GEMM.  The tiled launch is checked against the raw one over all outputs.  The
first 1 000 000 rows of the same bytes, read as a MatMul B [K = 1 000 000, N = 4096]
(blocks along N), are multiplied at 1, 8 and 64 rows of A and checked on two whole
column blocks (the first and the last).  Over a million-term K sum the reference's own
sequential fp32 chain (cpu_kernels.cpp:116-130) strays from the exact sum by ~1e-5
relative L2 (its error grows as the square root of K), so the bar is taken against the
exact product instead: float64 sums of the reference's element values d * q (the
oracle's dequantisation), relative L2 1e-5, with the oracle's restatement held to 1e-4
of the same exact product (B past 2 GiB keeps the FP32 MatMul kernel at every M).  The
Embedding gathers the first and last rows and out-of-range ids, from both layouts, bit
for bit against the oracle (cpu_kernels.cpp:286-295; ids outside the table give zero
rows, as the reference device kernel does, cuda_kernels.cu:399-427).
"""
import numpy as np
import pytest

from helpers import assert_bitexact, note
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu

N_BIG = 1_000_003
K_BIG = 4096
ROW_BYTES = K_BIG // 32 * 34


@pytest.fixture(scope="module")
def big_weight(dev):
    """(raw [N, K/32 * 34] uint8, tiled copy) on the device; int8 quants uniform in
    [-127, 127], binary16 scales |U(0, 1)| * 0.02 / 127, generated in row chunks."""
    import torch
    note(f"large weight: generating {N_BIG} x {K_BIG} Q8_0 ({N_BIG * ROW_BYTES / 2**30:.2f} GiB)")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261202)
    KB = K_BIG // 32
    w = torch.empty((N_BIG, KB, 34), dtype=torch.uint8, device=dev)
    for r0 in range(0, N_BIG, 65536):
        n = min(65536, N_BIG - r0)
        q = torch.randint(-127, 128, (n, KB, 32), dtype=torch.int16, device=dev, generator=gen)
        w[r0:r0 + n, :, 2:] = q.to(torch.int8).view(torch.uint8)
        d = (torch.rand((n, KB), device=dev, generator=gen) * (0.02 / 127)).to(torch.float16)
        w[r0:r0 + n, :, :2] = d.view(torch.uint8).view(n, KB, 2)
        del q, d
    w = w.view(-1)
    assert w.numel() > 2**32
    t = torch.empty(capi.tiled_bytes(N_BIG, K_BIG), dtype=torch.uint8, device=dev)
    capi.tile(w, t, N_BIG, K_BIG)
    torch.cuda.synchronize()
    yield w, t
    del w, t
    torch.cuda.empty_cache()


def _sample_rows(seed):
    rng = np.random.default_rng(seed)
    fixed = [0, 1, 15, 16, N_BIG // 2, N_BIG - 17, N_BIG - 4, N_BIG - 3, N_BIG - 2, N_BIG - 1]
    return np.unique(np.concatenate([fixed, rng.integers(0, N_BIG, size=40)])).astype(np.int64)


def _host_rows(w, rows):
    import torch
    idx = torch.as_tensor(rows, device=w.device)
    return w.view(N_BIG, ROW_BYTES).index_select(0, idx).cpu().numpy().reshape(-1)


@pytest.mark.parametrize("M", [1, 4, 8, 64])
def test_linear_weight_past_4gib(dev, orc, big_weight, M):
    import torch
    w, t = big_weight
    note(f"large weight Linear: M={M} N={N_BIG} K={K_BIG} (raw and tiled)")
    x = S.activations(4100 + M, (M, K_BIG))
    bias = S.activations(4200 + M, (N_BIG,), tag=S.TAG_BIAS) if M in (1, 64) else None
    dx = torch.from_numpy(x).to(dev)
    db = torch.from_numpy(bias).to(dev) if bias is not None else None
    y_raw = torch.full((M, N_BIG), float("nan"), dtype=torch.float32, device=dev)
    y_t = torch.full((M, N_BIG), float("nan"), dtype=torch.float32, device=dev)
    capi.linear(dx, w, db, y_raw, M, N_BIG, K_BIG)
    capi.linear_tiled(dx, t, db, y_t, M, N_BIG, K_BIG)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y_raw).all()) and bool(torch.isfinite(y_t).all())
    bar = 1e-2 if M >= 64 else 1e-5
    rows = _sample_rows(M)
    want = orc.linear(x, _host_rows(w, rows), bias[rows] if bias is not None else None, M,
                      rows.size, K_BIG)
    idx = torch.as_tensor(rows, device=dev)
    for name, y in (("raw", y_raw), ("tiled", y_t)):
        got = y.index_select(1, idx).cpu().numpy().astype(np.float64)
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert err <= bar, (name, err)
    diff = torch.linalg.vector_norm((y_t - y_raw).double()) / torch.linalg.vector_norm(y_raw.double())
    assert float(diff) <= (1e-2 if M >= 64 else 1e-6)


def test_embedding_table_past_4gib(dev, orc, big_weight):
    import torch
    w, t = big_weight
    ids = np.array([0, N_BIG - 1, 1, N_BIG - 2, -1, N_BIG, 123_457, N_BIG // 2, 999_999,
                    N_BIG - 17, 2**31 - 1, 15, 16], np.int32)
    n = ids.size
    note(f"large weight Embedding: vocab={N_BIG} hidden={K_BIG} n={n} (raw and tiled)")
    valid = (ids >= 0) & (ids < N_BIG)
    rows = np.unique(ids[valid]).astype(np.int64)
    local = np.full(n, -1, np.int32)
    local[valid] = np.searchsorted(rows, ids[valid]).astype(np.int32)
    want = orc.embedding_zero_fill(_host_rows(w, rows), local, rows.size, K_BIG)
    dids = torch.from_numpy(ids).to(dev)
    out = torch.full((n, K_BIG), float("nan"), dtype=torch.float32, device=dev)
    capi.embedding(w, dids, out, n, N_BIG, K_BIG)
    torch.cuda.synchronize()
    assert_bitexact(out.cpu().numpy(), want)
    out.fill_(float("nan"))
    capi.embedding_tiled(t, dids, out, n, N_BIG, K_BIG)
    torch.cuda.synchronize()
    assert_bitexact(out.cpu().numpy(), want)


@pytest.mark.parametrize("M", [1, 8, 64])
def test_matmul_b_past_4gib(dev, orc, big_weight, M):
    import torch
    w, _ = big_weight
    K, N = 1_000_000, K_BIG
    b = w[:K * ROW_BYTES]  # B [K, N] row-major, blocks along N: the weight's first K rows
    note(f"large weight MatMul: M={M} N={N} K={K}")
    a = S.activations(4300 + M, (M, K))
    da = torch.from_numpy(a).to(dev)
    c = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    capi.matmul(da, b, c, M, N, K)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(c).all())
    blocks = torch.tensor([0, N // 32 - 1], device=dev)
    b_sub = b.view(K, N // 32, 34).index_select(1, blocks).cpu().numpy().reshape(-1)
    exact = a.astype(np.float64) @ orc.dequantize_q8_0(b_sub, K * 64).reshape(K, 64).astype(
        np.float64)
    got = torch.cat([c[:, :32], c[:, N - 32:]], dim=1).cpu().numpy().astype(np.float64)
    err = np.linalg.norm(got - exact) / np.linalg.norm(exact)
    assert err <= 1e-5, err
    ref = orc.sgemm(a, b_sub, M, 64, K).astype(np.float64)
    ref_err = np.linalg.norm(ref - exact) / np.linalg.norm(exact)
    note(f"large MatMul M={M}: relative L2 to the exact product {err:.2e} (reference chain "
         f"{ref_err:.2e})")
    assert ref_err <= 1e-4, ref_err
