"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (stated per test): Embedding and MatMul bit-exact; Linear on the FP32 GEMV path
(M <= 63) relative L2 <= 1e-5; Linear on the bf16-MFMA path (M >= 64) relative L2
<= 1e-2.  The benchmark's full sizes are covered either directly against the oracle (where it
finishes in seconds) or through size-independent properties (agreement of the two
Linear paths, determinism, linearity).
"""
import functools

import numpy as np
import pytest

from helpers import (assert_bitexact, bits, empty_f32, hybrid_decode, note, rel_l2, sha,
                     to_dev, to_host)
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
MFMA_TOL = 1e-2


@functools.lru_cache(maxsize=None)
def weight(seed, rows, cols):
    w, _, _ = S.q8_0_weight(seed, rows, cols)
    return w


@functools.lru_cache(maxsize=None)
def acts(seed, rows, cols, tag=S.TAG_X):
    return S.activations(seed, (rows, cols), tag=tag)


def run_linear(dev, x, w, bias, M, N, K, path=0, **shape):
    dx, dw = to_dev(x, dev), to_dev(w, dev)
    db = to_dev(bias, dev) if bias is not None else None
    dy = empty_f32((M, N), dev)
    if path == 0 and not shape:
        capi.linear(dx, dw, db, dy, M, N, K)
    else:
        capi.linear_ex(dx, dw, db, dy, M, N, K, path=path, **shape)
    return to_host(dy)


# ----------------------------------------------------------------------------- decode

def test_f16_scale_decode_exhaustive(dev, orc):
    import torch
    note("f16 decode, all 65536 patterns")
    pat = torch.arange(65536, dtype=torch.int32, device=dev).to(torch.int16).view(torch.uint16)
    out = empty_f32((65536,), dev)
    capi.f16_decode(pat, out, 65536)
    got = to_host(out)
    want = orc.f16_table()
    assert np.array_equal(bits(got), bits(want))  # NaNs canonicalised like the reference


# ----------------------------------------------------------------------------- embedding

def test_embedding_known_answers(dev, orc, golden):
    for c in golden["cases"]:
        if not (c.get("known_answer") and c["op"] == "embedding"):
            continue
        note(c["name"])
        Q = np.array(c["quants"], np.int8)
        table = S.pack_q8_0_const_scale(Q, c["scale_bits"])
        ids = np.array(c["ids"], np.int32)
        out = empty_f32((ids.size, c["hidden"]), dev)
        capi.embedding(to_dev(table, dev), to_dev(ids, dev), out, ids.size, c["vocab"], c["hidden"])
        got = to_host(out)
        assert sha(got) == c["sha256"]


def test_embedding_c5_full_bitexact(dev, orc, golden):
    """Config 5: table [151936, 896], 8 x 512 ids; every output bit checked."""
    c = next(c for c in golden["cases"] if c["name"] == "embedding_c5_151936x896_4096")
    note("embedding C5 full")
    w = weight(c["seed"], c["vocab"], c["hidden"])
    ids = S.token_ids(c["seed"], c["n_ids"], c["vocab"])
    out = empty_f32((ids.size, c["hidden"]), dev)
    capi.embedding(to_dev(w, dev), to_dev(ids, dev), out, ids.size, c["vocab"], c["hidden"])
    got = to_host(out)
    assert_bitexact(got, orc.embedding(w, ids, c["hidden"]), "C5")
    assert sha(got) == c["sha256"]


@pytest.mark.parametrize("vocab,hidden,n", [(1, 32, 1), (3, 32, 7), (257, 64, 100),
                                            (1000, 896, 513), (77, 4096, 33)])
def test_embedding_ragged_bitexact(dev, orc, vocab, hidden, n):
    note(f"embedding vocab={vocab} hidden={hidden} n={n}")
    w = weight(50 + vocab, vocab, hidden)
    ids = S.token_ids(51 + n, n, vocab)
    ids[-1] = vocab - 1  # always touch the last row, the last bytes of the table
    out = empty_f32((n, hidden), dev)
    capi.embedding(to_dev(w, dev), to_dev(ids, dev), out, n, vocab, hidden)
    assert_bitexact(to_host(out), orc.embedding(w, ids, hidden))


def test_embedding_out_of_range_ids_give_zero_rows(dev, orc):
    vocab, hidden = 40, 64
    w = weight(52, vocab, hidden)
    ids = np.array([3, -1, 39, 40, 7, 2 ** 31 - 1, -2 ** 31, 0], np.int32)
    note("embedding invalid ids")
    out = empty_f32((ids.size, hidden), dev)
    capi.embedding(to_dev(w, dev), to_dev(ids, dev), out, ids.size, vocab, hidden)
    assert_bitexact(to_host(out), orc.embedding_zero_fill(w, ids, vocab, hidden))


def test_embedding_special_scales(dev, orc):
    """Every binary16 class as a scale, with signed zeros: bit-exact except that
    NaN outputs are compared by position (x86 and AMD differ on the sign of the
    NaN produced by Inf * 0)."""
    specials = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0x7BFF,
                         0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE00, 0x13FF, 0x8200],
                        np.uint16)
    q = S.quants(53, specials.size * 32)
    q[::7] = 0
    table = S.pack_q8_0(q, specials.view(np.float16))
    ids = np.arange(specials.size, dtype=np.int32)[::-1].copy()
    note("embedding special scales")
    out = empty_f32((ids.size, 32), dev)
    capi.embedding(to_dev(table, dev), to_dev(ids, dev), out, ids.size, specials.size, 32)
    assert_bitexact(to_host(out), orc.embedding(table, ids, 32))


def _tiled_table(table, vocab, hidden, dev):
    import torch
    dw = to_dev(table, dev)
    t = torch.empty(capi.tiled_bytes(vocab, hidden), dtype=torch.uint8, device=dev)
    capi.tile(dw, t, vocab, hidden)
    return t


@pytest.mark.parametrize("vocab,hidden,n", [(1, 32, 1), (3, 96, 7), (257, 64, 100),
                                            (1000, 896, 513), (77, 4096, 33),
                                            (151936, 896, 4096)])
def test_embedding_tiled_table_bitexact(dev, orc, vocab, hidden, n):
    """The gather from a table in 16-row tiles equals the reference gather bit for
    bit: ragged vocabularies (rows past the last 16-row group), hidden with an odd
    number of blocks (96: the pair's second block is padding), out-of-range ids
    (zero rows), the configs[4] shape."""
    note(f"embedding tiled vocab={vocab} hidden={hidden} n={n}")
    w = weight(60 + vocab, vocab, hidden)
    ids = S.token_ids(61 + n, n, vocab)
    ids[-1] = vocab - 1
    if n > 4:
        ids[1], ids[2] = -1, vocab
    out = empty_f32((n, hidden), dev)
    capi.embedding_tiled(_tiled_table(w, vocab, hidden, dev), to_dev(ids, dev), out, n, vocab,
                         hidden)
    assert_bitexact(to_host(out), orc.embedding_zero_fill(w, ids, vocab, hidden))


def test_embedding_tiled_table_special_scales(dev, orc):
    """Every binary16 class as a scale through the tiled table (NaN outputs by position)."""
    specials = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0x7BFF,
                         0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE00, 0x13FF, 0x8200,
                         0x3555, 0x0200], np.uint16)
    hidden = 64
    q = S.quants(54, specials.size * hidden)
    q[::7] = 0
    table = S.pack_q8_0(q, np.repeat(specials, hidden // 32).view(np.float16))
    vocab = specials.size
    ids = np.arange(vocab, dtype=np.int32)[::-1].copy()
    note("embedding tiled special scales")
    out = empty_f32((ids.size, hidden), dev)
    capi.embedding_tiled(_tiled_table(table, vocab, hidden, dev), to_dev(ids, dev), out,
                         ids.size, vocab, hidden)
    assert_bitexact(to_host(out), orc.embedding(table, ids, hidden))


def test_embedding_tiled_table_errors(dev):
    import torch
    w = _tiled_table(weight(55, 16, 64), 16, 64, dev)
    ids = to_dev(np.zeros(2, np.int32), dev)
    out = empty_f32((2, 64), dev)
    code, msg = capi.embedding_tiled_status(w, ids, out, 2, 16, 48)
    assert code == 4 and "multiple of 32" in msg
    unaligned = torch.empty(w.numel() + 16, dtype=torch.uint8, device=dev)[8:]
    code, msg = capi.embedding_tiled_status(unaligned, ids, out, 2, 16, 64)
    assert code == 1 and "aligned" in msg
    code, msg = capi.embedding_tiled_status(w, ids, out, -1, 16, 64)
    assert code == 1


def test_embedding_empty_is_noop(dev):
    w = to_dev(weight(54, 4, 32), dev)
    ids = to_dev(np.zeros(1, np.int32), dev)
    out = empty_f32((1, 32), dev)
    capi.embedding(w, ids, out, 0, 4, 32)
    assert np.all(np.isnan(to_host(out)))


@pytest.mark.parametrize("rows,cols,cut", [(151936, 896, 0), (4096, 4096, 0), (77, 96, 5),
                                           (1, 32, 31), (3, 64, 0)])
def test_dequantize_bitexact(dev, orc, rows, cols, cut):
    """Loader Q8_0 -> fp32 on the device against the oracle's whole-stream dequantisation,
    bit for bit; `cut` elements short of whole blocks exercises the partial last block."""
    note(f"dequantize {rows}x{cols} - {cut}")
    w, _, _ = S.q8_0_weight(140 + cols, rows, cols)
    n = rows * cols - cut
    out = empty_f32((n,), dev)
    capi.dequantize(to_dev(w, dev), out, n)
    assert_bitexact(to_host(out), orc.dequantize_q8_0(w, n), "dequantize")


def test_dequantize_special_scales_and_errors(dev, orc):
    import torch
    special = np.array([0x0001, 0x03ff, 0x0000, 0x8000, 0x7c00, 0xfc00, 0x7e00, 0x3c00] * 4,
                       dtype=np.uint16)
    w, _, _ = S.q8_0_weight(150, 32, 32)
    w = w.copy()
    w.reshape(32, 34)[:, :2] = special.view(np.uint8).reshape(32, 2)
    out = empty_f32((32 * 32,), dev)
    capi.dequantize(to_dev(w, dev), out, 32 * 32)
    assert_bitexact(to_host(out), orc.dequantize_q8_0(w, 32 * 32), "special scales")
    capi.dequantize(to_dev(w, dev), out, 0)  # no-op
    code, msg = capi.dequantize_status(None, out, 4)
    assert code == 1 and "src pointer" in msg
    code, msg = capi.dequantize_status(to_dev(w, dev), out[1:], 4)
    assert code == 1 and "16-byte aligned" in msg
    code, msg = capi.dequantize_status(to_dev(w, dev), out, -1)
    assert code == 1 and "negative" in msg
    torch.cuda.synchronize()


# ----------------------------------------------------------------------------- linear GEMV

def test_linear_known_answers_exact(dev, golden):
    """Integer quants x dyadic activations: every partial sum is exact, so the GPU
    must reproduce the reference's bits whatever its summation order."""
    for c in golden["cases"]:
        if not (c.get("known_answer") and c["op"] == "linear"):
            continue
        note(c["name"])
        Q = np.array(c["quants"], np.int8)
        w = S.pack_q8_0_const_scale(Q, c["scale_bits"])
        x = np.array(c["activations"], np.float32).reshape(c["M"], c["K"])
        # path 1 FP32 GEMV, 3 MFMA decode (exact bf16 parts), 2 bf16 MFMA GEMM
        # (dyadic inputs with <= 8 significant bits stay exact there too)
        for path in (1, 2, 3):
            got = run_linear(dev, x, w, None, c["M"], c["N"], c["K"], path=path)
            assert sha(got) == c["sha256"], (c["name"], path)


def test_linear_c1_full(dev, orc):
    M, N, K = 1, 4096, 4096
    note("linear C1 1x4096x4096")
    w, x = weight(1, N, K), acts(1, M, K)
    got = run_linear(dev, x, w, None, M, N, K)
    assert rel_l2(got, orc.sgemm_nt(x, w, M, N, K)) <= GEMV_TOL


C2_SHAPES = [(12288, 4096), (4096, 4096), (11008, 4096), (4096, 11008)]


@pytest.mark.parametrize("M", [1, 4, 8])
@pytest.mark.parametrize("N,K", C2_SHAPES)
def test_linear_c2_llama_decode(dev, orc, M, N, K):
    note(f"linear C2 M={M} N={N} K={K}")
    w, x = weight(2, N, K), acts(2 + M, M, K)
    got = run_linear(dev, x, w, None, M, N, K)
    err = rel_l2(got, orc.sgemm_nt(x, w, M, N, K))
    assert err <= GEMV_TOL, err


@pytest.mark.parametrize("N,K,M", [(1152, 896, 1), (4864, 896, 1), (896, 4864, 1),
                                   (151936, 896, 1), (151936, 896, 8), (1152, 896, 4),
                                   (4864, 896, 2), (896, 4864, 3)])
def test_linear_c4_qwen_decode(dev, orc, N, K, M):
    note(f"linear C4 M={M} N={N} K={K}")
    w, x = weight(4, N, K), acts(4 + M, M, K)
    got = run_linear(dev, x, w, None, M, N, K)
    err = rel_l2(got, orc.sgemm_nt(x, w, M, N, K))
    assert err <= GEMV_TOL, err


@pytest.mark.parametrize("M,N,K", [(1, 1, 32), (2, 3, 64), (3, 7, 96), (5, 33, 992),
                                   (8, 1000, 512), (6, 129, 2080), (1, 515, 11008),
                                   (9, 40, 256), (17, 65, 1024), (63, 100, 320)])
def test_linear_ragged_with_bias(dev, orc, M, N, K):
    note(f"linear ragged M={M} N={N} K={K}")
    w, x = weight(60 + N, N, K), acts(61 + K, M, K)
    bias = S.activations(62, (N,), tag=S.TAG_BIAS)
    got = run_linear(dev, x, w, bias, M, N, K)
    err = rel_l2(got, orc.linear(x, w, bias, M, N, K))
    assert err <= GEMV_TOL, err


def test_linear_every_gemv_launch_shape(dev, orc):
    """All (mt, lpr, rw) instantiations on a ragged shape, M from 1 to mt."""
    N, K = 77, 1312
    w = weight(70, N, K)
    for mt in (1, 2, 4, 8):
        M = max(1, mt - 1) if mt > 1 else 1
        x = acts(71 + M, M, K)
        want = orc.sgemm_nt(x, w, M, N, K)
        for lpr in (16, 32, 64):
            for rw in (1, 2, 4, 8):
                note(f"gemv shape mt={mt} lpr={lpr} rw={rw} M={M}")
                got = run_linear(dev, x, w, None, M, N, K, path=1, mt=mt, lpr=lpr, rw=rw)
                assert rel_l2(got, want) <= GEMV_TOL, (mt, lpr, rw)


def test_linear_gemv_deterministic_and_linear(dev):
    """lm_head [151936, 896] at M=8: bitwise repeatable, and linear in x."""
    import torch
    N, K, M = 151936, 896, 8
    note("gemv determinism/linearity lm_head")
    dw = to_dev(weight(4, N, K), dev)
    x1, x2 = acts(80, M, K), acts(81, M, K)
    d1, d2, d12 = to_dev(x1, dev), to_dev(x2, dev), to_dev(x1 + x2, dev)
    y1a, y1b, y2, y12 = (empty_f32((M, N), dev) for _ in range(4))
    capi.linear(d1, dw, None, y1a, M, N, K)
    capi.linear(d1, dw, None, y1b, M, N, K)
    capi.linear(d2, dw, None, y2, M, N, K)
    capi.linear(d12, dw, None, y12, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y1a, y1b)
    assert rel_l2(to_host(y12), to_host(y1a) + to_host(y2)) <= GEMV_TOL


@pytest.mark.parametrize("N,K", [(12288, 4096), (11008, 4096), (4096, 4096), (8200, 2080)])
def test_linear_two_tokens_gemv(dev, orc, N, K):
    """M = 2 on raw weights with rows of 2048-4096 elements takes the FP32 GEMV
    (automatic path; two rows per lane group from 8192 outputs; 8200 x 2080: a ragged
    last row pair and 65 blocks per row): with bias, against the oracle, and bit-equal
    to the forced GEMV launch with one and with two rows per group (the row count
    does not change a row's sum)."""
    M = 2
    note(f"two-token GEMV {N}x{K}")
    w, x = weight(82, N, K), acts(83, M, K)
    bias = S.activations(84, (N,), tag=S.TAG_BIAS)
    want = orc.linear(x, w, bias, M, N, K)
    got = run_linear(dev, x, w, bias, M, N, K)
    assert rel_l2(got, want) <= GEMV_TOL
    for rw in (1, 2):
        forced = run_linear(dev, x, w, bias, M, N, K, path=1, mt=2, lpr=32, rw=rw)
        assert np.array_equal(bits(got), bits(forced)), rw


# (N, K, byte shift of W): Llama o_proj / down, a ragged row count with 65 blocks per
# row (the second 64-block chunk holds one live lane), the Qwen down projection (152
# blocks: a partial last chunk), 10 chunks of 64 blocks over 8 waves (the chunk loop),
# and W 2 bytes past a 4-byte boundary (every block at its other 4-byte phase).
RAWK_CASES = [(4096, 4096, 0), (4096, 11008, 0), (515, 2080, 2), (896, 4864, 0),
              (7, 20480, 2), (4096, 11008, 2)]


@pytest.mark.parametrize("N,K,shift", RAWK_CASES)
def test_linear_one_token_row_span(dev, orc, N, K, shift):
    """The row-span kernel (forced launch shape; the automatic path for one token on
    rows of more than 4096 elements): with bias, against the oracle; within 1e-6 of the
    LDS-staged GEMV; bitwise repeatable; a BFloat16 bias gives the widened fp32 bias's
    bits; bit-equal to the automatic path where that takes it."""
    import torch
    M = 1
    note(f"row-span GEMV {N}x{K} shift={shift}")
    w, x = weight(90 + N, N, K), acts(91 + K, M, K)
    b32 = S.activations(92, (N,), tag=S.TAG_BIAS)
    b16 = (b32.view(np.uint32) >> 16).astype(np.uint16)
    widened = (b16.astype(np.uint32) << 16).view(np.float32)
    dx, dw = to_dev(x, dev), to_dev(w, dev)
    if shift:
        buf = torch.zeros(dw.numel() + shift, dtype=torch.uint8, device=dev)
        buf[shift:] = dw
        dw = buf[shift:]
        assert dw.data_ptr() % 4 == shift
    db = to_dev(widened, dev)
    y, y2, y16, yold, auto = (empty_f32((M, N), dev) for _ in range(5))
    for out in (y, y2):
        capi.linear_ex(dx, dw, db, out, M, N, K, path=1, mt=1, rpw=4)
    capi.linear_bias_bf16(dx, dw, to_dev(b16, dev), y16, M, N, K)
    capi.linear_ex(dx, dw, db, yold, M, N, K, path=1, mt=1, lpr=64, rw=1)
    capi.linear(dx, dw, db, auto, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert torch.equal(auto, y16)
    got = to_host(y)
    assert rel_l2(got, orc.linear(x, w, widened, M, N, K)) <= GEMV_TOL
    assert rel_l2(got, to_host(yold)) <= 1e-6
    if K > 4096:
        assert torch.equal(y, auto)


def test_linear_multi_one_token_row_span(dev, orc):
    """A one-token multi-output Linear on rows of more than 4096 elements runs the
    row-span kernel over its three segments: each output against the oracle and
    bit-equal to its single Linear (the same kernel)."""
    import torch
    M, K, Ns = 1, 4864, (1000, 24, 3000)
    note(f"row-span multi {Ns} K={K}")
    x = acts(93, M, K)
    ws = [weight(94 + i, n, K) for i, n in enumerate(Ns)]
    bs = [S.activations(97 + i, (n,), tag=S.TAG_BIAS) for i, n in enumerate(Ns)]
    dx = to_dev(x, dev)
    dws = [to_dev(w, dev) for w in ws]
    dbs = [to_dev(b, dev) for b in bs]
    ys = [empty_f32((M, n), dev) for n in Ns]
    singles = [empty_f32((M, n), dev) for n in Ns]
    capi.linear_multi(dx, dws, dbs, ys, list(Ns), M, K)
    for dw, db, yy, n in zip(dws, dbs, singles, Ns):
        capi.linear(dx, dw, db, yy, M, n, K)
    torch.cuda.synchronize()
    for i, n in enumerate(Ns):
        assert torch.equal(ys[i], singles[i]), i
        assert rel_l2(to_host(ys[i]), orc.linear(x, ws[i], bs[i], M, n, K)) <= GEMV_TOL, i


# ----------------------------------------------------------------------------- linear MFMA decode

DECODE_SHAPES = [(2, 16), (4, 16), (8, 16), (2, 32), (4, 32), (8, 32)]


def test_linear_every_decode_mfma_shape(dev, orc):
    """All (mt, waves, kslice) instantiations of the MFMA decode kernel on a ragged
    shape (N = 77 rows, K = 1312: 41 blocks, so K splits into 3 or 2 slices and the
    last is partial), M from mt-1 to mt, with bias; then a shape with one slice."""
    w = weight(72, 77, 1312)
    bias = S.activations(73, (77,), tag=S.TAG_BIAS)
    for N, K in ((77, 1312), (77, 160)):
        wNK = w if K == 1312 else weight(72, N, K)
        for mt in (1, 2, 4, 5, 8, 16):
            for M in sorted({max(1, mt - 1), mt}):
                x = acts(74 + M, M, K)
                want = orc.linear(x, wNK, bias, M, N, K)
                for waves, kslice in DECODE_SHAPES:
                    if mt == 16 and kslice == 32:
                        continue
                    note(f"decode mfma mt={mt} waves={waves} kslice={kslice} M={M} K={K}")
                    got = run_linear(dev, x, wNK, bias, M, N, K, path=3, mt=mt, waves=waves,
                                     kslice=kslice)
                    assert rel_l2(got, want) <= GEMV_TOL, (mt, waves, kslice, M, K)


@pytest.mark.parametrize("M", [2, 3, 5, 7, 16, 17, 40])
def test_linear_decode_mfma_sizes(dev, orc, M):
    """Automatic launch shapes for token counts between the tiles (and chunks of 16)."""
    N, K = 1000, 2080
    note(f"decode mfma M={M}")
    w, x = weight(75, N, K), acts(76 + M, M, K)
    got = run_linear(dev, x, w, None, M, N, K, path=3)
    err = rel_l2(got, orc.sgemm_nt(x, w, M, N, K))
    assert err <= GEMV_TOL, err


def test_linear_decode_mfma_exact_parts_wide_range(dev, orc):
    """Activations spanning 2^-60 .. 2^60 and values with all 24 significand bits
    set: the three bf16 parts carry every bit, so the error stays at fp32
    accumulation level (checked per token against the oracle)."""
    M, N, K = 4, 96, 512
    w = weight(77, N, K)
    rng = np.random.default_rng(7)
    mant = (1.0 + rng.integers(0, 1 << 23, size=(M, K)) / float(1 << 23)).astype(np.float64)
    expo = rng.integers(-60, 61, size=(M, K))
    sign = np.where(rng.integers(0, 2, size=(M, K)) == 1, -1.0, 1.0)
    x = (sign * mant * np.exp2(expo)).astype(np.float32)
    x[1] = (x[1] / 1e30).astype(np.float32)  # one token entirely tiny
    note("decode mfma wide-range activations")
    got = run_linear(dev, x, w, None, M, N, K, path=3)
    want = orc.sgemm_nt(x, w, M, N, K)
    for m in range(M):
        assert rel_l2(got[m], want[m]) <= GEMV_TOL, m


def test_linear_decode_mfma_nonfinite_activations(dev, orc):
    """+-Inf and NaN activations propagate as in the reference's FP32 FMA chain:
    same NaN positions, same signed infinities, finite values within 1e-5."""
    M, N, K = 4, 130, 256
    w = weight(78, N, K)
    x = acts(79, M, K).copy()
    x[0, 5] = np.inf
    x[1, 40] = -np.inf
    x[2, 7] = np.nan
    x[3, 100] = np.inf
    x[3, 101] = -np.inf
    note("decode mfma non-finite activations")
    got = run_linear(dev, x, w, None, M, N, K, path=3)
    want = orc.sgemm_nt(x, w, M, N, K)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.sign(got[np.isinf(want)]), np.sign(want[np.isinf(want)]))
    assert rel_l2(got[fin], want[fin]) <= GEMV_TOL


def test_linear_decode_mfma_split_k_deterministic(dev):
    """QKV [12288, 4096] at M=8 runs 8 K splits: repeated launches are bitwise
    identical (partials are added in split order), and equal across streams."""
    import torch
    M, N, K = 8, 12288, 4096
    note("decode mfma split-K determinism")
    dw, dx = to_dev(weight(2, N, K), dev), to_dev(acts(2 + M, M, K), dev)
    ya, yb = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear(dx, dw, None, ya, M, N, K)
    for _ in range(3):
        capi.linear(dx, dw, None, yb, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(ya, yb)
    s2 = torch.cuda.Stream()
    yc = empty_f32((M, N), dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(s2):
        capi.linear(dx, dw, None, yc, M, N, K, stream=s2)
    torch.cuda.synchronize()
    assert torch.equal(ya, yc)


def test_linear_decode_mfma_two_streams_concurrently(dev, orc):
    """Two streams, each with its own split-K workspace, interleaving launches of
    different shapes; every result matches the oracle."""
    import torch
    note("decode mfma two streams")
    shapes = [(8, 4096, 4096), (4, 1024, 11008)]
    data = []
    for i, (M, N, K) in enumerate(shapes):
        w, x = weight(120 + i, N, K), acts(121 + i, M, K)
        data.append((M, N, K, w, x, to_dev(w, dev), to_dev(x, dev),
                     [empty_f32((M, N), dev) for _ in range(4)]))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for j in range(4):
        for (M, N, K, _, _, dw, dx, ys), s in zip(data, streams):
            capi.linear(dx, dw, None, ys[j], M, N, K, stream=s)
    torch.cuda.synchronize()
    for M, N, K, w, x, _, _, ys in data:
        want = orc.sgemm_nt(x, w, M, N, K)
        for y in ys:
            assert rel_l2(to_host(y), want) <= GEMV_TOL


def test_linear_decode_mfma_split_k_after_poisoned_workspace(dev, orc):
    """The split-K hand-off reads only partials written by its own launch: before each
    launch with K splits, a launch of another shape on the same stream fills the same
    workspace lines with NaN partials (NaN activations, 16 tokens, 22 splits of the
    split-K kernel: 5.8 MB of partials).  Every result of the split-K kernel (8 and 22
    splits) and of the hybrid decode (8 splits of 44 blocks at 4 tokens, 6 at 8 tokens;
    raw and tiled weights) stays finite and within 1e-5 relative L2 of the oracle."""
    import torch
    Mp, Np, Kp = 16, 4096, 11008
    xp = np.full((Mp, Kp), np.nan, dtype=np.float32)
    dwp, dxp = to_dev(weight(130, Np, Kp), dev), to_dev(xp, dev)
    yp = empty_f32((Mp, Np), dev)
    cases = [(8, 4096, 4096, False), (16, 4096, 11008, False), (4, 4096, 11008, False),
             (8, 4096, 8192, True)]
    assert hybrid_decode(4, 4096, 11008) and hybrid_decode(8, 4096, 8192)
    for M, N, K, tiled in cases:
        note(f"K splits after poisoned workspace M={M} N={N} K={K} tiled={tiled}")
        w, x = weight(131 + K, N, K), acts(132 + M, M, K)
        want = orc.sgemm_nt(x, w, M, N, K)
        dw, dx = to_dev(w, dev), to_dev(x, dev)
        if tiled:
            dwt = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
            capi.tile(dw, dwt, N, K)
            dw = dwt
        lin = capi.linear_tiled if tiled else capi.linear
        for _ in range(3):
            capi.linear(dxp, dwp, None, yp, Mp, Np, Kp)     # NaN partials everywhere
            y = empty_f32((M, N), dev)
            lin(dx, dw, None, y, M, N, K)
            torch.cuda.synchronize()
            got = to_host(y)
            assert np.isfinite(got).all()
            assert rel_l2(got, want) <= GEMV_TOL
        assert np.isnan(to_host(yp)).all()


def test_linear_threads_share_one_stream_while_workspace_grows(dev, orc):
    """Host threads launching on one (new) stream while its workspace grows: each
    thread runs shapes of increasing workspace need (split-K decode with 8 splits,
    0.26 MB; with 22 splits at 16 tokens, 5.8 MB; the prefill GEMM with its bf16 copy
    of X, 19.7 MB), starting from the 4 MB first allocation, so calls replace the
    buffers other threads have just taken (the replaced ones stay allocated for the
    launches already enqueued).  The workspace table stays locked until a launch is
    enqueued, so every result equals the oracle's (decode 1e-5, GEMM 1e-2) and the
    workspace ends at the largest need, after at least one replacement."""
    import threading
    import torch
    shapes = [(8, 1024, 4096), (16, 4096, 11008), (512, 1024, 11008)]
    data = []
    for i, (M, N, K) in enumerate(shapes):
        w, x = weight(140 + i, N, K), acts(141 + i, M, K)
        data.append((M, N, K, to_dev(w, dev), to_dev(x, dev), orc.sgemm_nt(x, w, M, N, K)))
    stream = torch.cuda.Stream()
    T, R = 3, 4
    outs = [[[empty_f32((M, N), dev) for (M, N, K, *_r) in data] for _ in range(R)]
            for _ in range(T)]
    errors = []

    def work(t):
        try:
            for r in range(R):
                for i, (M, N, K, dw, dx, _) in enumerate(data):
                    capi.linear(dx, dw, None, outs[t][r][i], M, N, K, stream=stream)
        except Exception as e:  # surfaced below
            errors.append(e)

    torch.cuda.synchronize()  # inputs and outputs are in place before any launch
    M0, N0, K0, dw0, dx0, _ = data[0]
    capi.linear(dx0, dw0, None, empty_f32((M0, N0), dev), M0, N0, K0, stream=stream)
    stream.synchronize()
    gen0 = capi.workspace_info(stream)[2]  # the first (4 MB) allocation
    assert gen0 >= 1
    note("threads share one stream while its workspace grows")
    threads = [threading.Thread(target=work, args=(t,)) for t in range(T)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    stream.synchronize()
    assert not errors, errors
    for t in range(T):
        for r in range(R):
            for i, (M, N, K, _dw, _dx, want) in enumerate(data):
                bar = MFMA_TOL if M >= 64 else GEMV_TOL
                assert rel_l2(to_host(outs[t][r][i]), want) <= bar, (t, r, i)
    need = [capi.workspace_size(capi.OP_LINEAR, M, [N], K) for (M, N, K, *_r) in data]
    b, c, g = capi.workspace_info(stream)
    assert b >= max(n[0] for n in need) and c >= max(n[1] for n in need)
    assert g > gen0  # the larger shapes replaced the first buffer


# ----------------------------------------------------------------------------- linear MFMA

@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (65, 130, 96), (128, 128, 128),
                                   (200, 333, 512), (64, 1, 32), (300, 257, 4096)])
def test_linear_mfma_ragged_with_bias(dev, orc, M, N, K):
    note(f"mfma ragged M={M} N={N} K={K}")
    w, x = weight(90 + N, N, K), acts(91 + K, M, K)
    bias = S.activations(92, (N,), tag=S.TAG_BIAS)
    got = run_linear(dev, x, w, bias, M, N, K)
    err = rel_l2(got, orc.linear(x, w, bias, M, N, K))
    assert err <= MFMA_TOL, err


def test_linear_mfma_split_k(dev, orc):
    """The prefill GEMM with its K split 1..5 ways (ragged M, N and K, bias):
    every split count agrees with the oracle, and repeats are bitwise equal."""
    import torch
    M, N, K = 200, 333, 1312
    w, x = weight(93, N, K), acts(94, M, K)
    bias = S.activations(95, (N,), tag=S.TAG_BIAS)
    want = orc.linear(x, w, bias, M, N, K)
    dx, dw, db = to_dev(x, dev), to_dev(w, dev), to_dev(bias, dev)
    for splits in (1, 2, 3, 5):
        note(f"mfma split-K splits={splits}")
        ya, yb = empty_f32((M, N), dev), empty_f32((M, N), dev)
        capi.linear_ex(dx, dw, db, ya, M, N, K, path=2, splits=splits)
        capi.linear_ex(dx, dw, db, yb, M, N, K, path=2, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(ya, yb)
        assert rel_l2(to_host(ya), want) <= MFMA_TOL, splits


@pytest.mark.parametrize("N,K", [(11008, 4096), (4096, 11008)])
def test_linear_c3_prefill_full(dev, orc, N, K):
    """Config 3 at full size (M=512): sampled rows against the oracle, the whole
    output against the FP32 GEMV path (itself pinned to the oracle at 1e-5)."""
    import torch
    M = 512
    note(f"mfma C3 M={M} N={N} K={K}")
    w, x = weight(3, N, K), acts(3, M, K)
    dx, dw = to_dev(x, dev), to_dev(w, dev)
    y_mfma, y_fp32 = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear(dx, dw, None, y_mfma, M, N, K)
    capi.linear_ex(dx, dw, None, y_fp32, M, N, K, path=1)
    torch.cuda.synchronize()
    got, fp32 = to_host(y_mfma), to_host(y_fp32)
    rows = np.array([0, 1, 255, 511])
    want_rows = orc.sgemm_nt(x[rows], w, rows.size, N, K)
    assert rel_l2(fp32[rows], want_rows) <= GEMV_TOL
    assert rel_l2(got[rows], want_rows) <= MFMA_TOL
    assert rel_l2(got, fp32) <= MFMA_TOL
    y_again = empty_f32((M, N), dev)
    capi.linear(dx, dw, None, y_again, M, N, K)
    assert torch.equal(y_again, y_mfma)


# ----------------------------------------------------------------------------- matmul

def test_matmul_known_answers(dev, golden):
    for c in golden["cases"]:
        if not (c.get("known_answer") and c["op"] == "matmul"):
            continue
        if c["K"] % 32:
            continue  # the device path requires K % 32 == 0 (cuda_kernels.cu:856-858)
        note(c["name"])
        Q = np.array(c["quants"], np.int8)
        b = S.pack_q8_0_const_scale(Q, c["scale_bits"])
        a = np.array(c["activations"], np.float32).reshape(c["M"], c["K"])
        out = empty_f32((c["M"], c["N"]), dev)
        capi.matmul(to_dev(a, dev), to_dev(b, dev), out, c["M"], c["N"], c["K"])
        assert sha(to_host(out)) == c["sha256"]


# (M, N, K) of the FP32 MatMul (M < 64): 1, 2, 4 and 8 token rows per tile (a partial
# last tile at M = 3, 5, 33, 63); N past a 256-column tile (ragged tiles) and an odd
# number of blocks per B row (rows alternate 4-byte phase: N = 32, 96); K past a
# 256-row slice; shapes whose K is spread over several workgroups (the workspace path:
# 1 x 4096 x 4096 and 4 x 11008 x 4096 with the last-arriving workgroup adding the
# partials, 2 x 512 x 11008 with 43 of them) and shapes whose column tiles alone fill
# the GPU.
MATMUL_CASES = [(2, 32, 32), (3, 64, 160), (5, 256, 512), (1, 32, 4096), (8, 1024, 96),
                (33, 96, 64), (4, 32, 32), (63, 512, 256), (1, 4096, 4096),
                (2, 512, 11008), (9, 800, 288), (1, 151936, 64), (3, 96, 1024),
                (8, 4096, 4096), (4, 11008, 4096)]


@pytest.mark.parametrize("M,N,K", MATMUL_CASES)
def test_matmul_matches_oracle(dev, orc, M, N, K):
    """Against the reference CPU kernel's arithmetic (cpu_kernels.cpp:116-130): the
    device adds the K sum in fixed pieces, so within fp32 rounding of the sequential
    sum (relative L2 <= 1e-5, the decode bar) and repeatable bit for bit."""
    import torch
    note(f"matmul M={M} N={N} K={K}")
    b, a = weight(100 + N, K, N), acts(101 + K, M, K)
    out, out2 = empty_f32((M, N), dev), empty_f32((M, N), dev)
    da, db = to_dev(a, dev), to_dev(b, dev)
    capi.matmul(da, db, out, M, N, K)
    capi.matmul(da, db, out2, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    got, want = to_host(out), orc.sgemm(a, b, M, N, K)
    assert rel_l2(got, want) <= 1e-5, (M, N, K)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("M,N,K", [(1, 96, 256), (4, 4096, 512), (8, 512, 1024), (2, 32, 64)])
def test_matmul_b_at_two_byte_offset(dev, M, N, K):
    """B may start 2 bytes past a 4-byte boundary (Q8_0 blocks are 34 bytes): every
    block then sits at the other 4-byte phase, so the up-to-8-row kernel takes its
    other load pattern; the result is the aligned copy's bit for bit."""
    import torch
    b, a = weight(400 + N, K, N), acts(401 + K, M, K)
    da, db = to_dev(a, dev), to_dev(b, dev)
    buf = torch.zeros(db.numel() + 2, dtype=torch.uint8, device=dev)
    buf[2:] = db
    shifted = buf[2:]
    assert shifted.data_ptr() % 4 == 2
    out, out2 = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.matmul(da, db, out, M, N, K)
    capi.matmul(da, shifted, out2, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), out2.view(torch.int32)), (M, N, K)


# (M, N, K) of the MatMul on the bf16 MFMA GEMM (M >= 64): the configs[2]-sized square
# shape, ragged M / N tiles with an odd number of K blocks (the last K step half empty),
# the smallest GEMM shape, a long K with split-K partials, and two shapes on 256-row
# tiles (taken where they fit the grid in one round and 128-row tiles do not), one with
# a ragged second row tile and an odd number of K blocks.
MATMUL_GEMM_CASES = [(512, 4096, 4096), (77, 1056, 1312), (64, 32, 32), (130, 384, 11008),
                     (512, 11008, 512), (300, 11264, 352)]


@pytest.mark.parametrize("M,N,K", MATMUL_GEMM_CASES)
def test_matmul_gemm_path(dev, orc, M, N, K):
    """MatMul from 64 rows of A runs the bf16 MFMA GEMM with B[K, N] dequantised
    transposed into its W tile.  Bar 1e-2 relative L2 (the prefill GEMM's): against the
    oracle's cpu::sgemm restatement (cpu_kernels.cpp:116-130) on sampled rows, and on the
    whole output against the FP32 MatMul run on 32-row chunks (the M < 64 path, held to
    1e-5 by test_matmul_matches_oracle); repeatable bit for bit."""
    import torch
    note(f"matmul GEMM M={M} N={N} K={K}")
    b, a = weight(300 + N, K, N), acts(301 + K, M, K)
    out, out2 = empty_f32((M, N), dev), empty_f32((M, N), dev)
    da, db = to_dev(a, dev), to_dev(b, dev)
    capi.matmul(da, db, out, M, N, K)
    capi.matmul(da, db, out2, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    got = to_host(out)
    assert np.isfinite(got).all()
    rows = np.unique(np.r_[0, M - 1, np.linspace(0, M - 1, 30).astype(int)])
    want = orc.sgemm(np.ascontiguousarray(a[rows]), b, rows.size, N, K)
    assert rel_l2(got[rows], want) <= 1e-2, (M, N, K)
    ref = empty_f32((M, N), dev)
    for m0 in range(0, M, 32):
        mc = min(32, M - m0)
        capi.matmul(da[m0:m0 + mc], db, ref[m0:m0 + mc], mc, N, K)
    fp32 = to_host(ref)
    assert rel_l2(fp32[rows], want) <= 1e-5
    assert rel_l2(got, fp32) <= 1e-2, (M, N, K)


# ----------------------------------------------------------------------------- errors

def test_device_error_paths(dev):
    x = to_dev(acts(110, 1, 64), dev)
    w = to_dev(weight(110, 2, 64), dev)
    y = empty_f32((1, 2), dev)
    code, msg = capi.linear_status(x, w, None, y, 1, 2, 31)
    assert code == 4 and "Q8_0" in msg and "32" in msg
    with pytest.raises(capi.Q8_0Error) as e:
        capi.matmul(x, w, y, 1, 2, 64)
    assert e.value.code == 4


# ----------------------------------------------------------------------------- BF16 bias

@pytest.mark.parametrize("M,N,K,tiled", [(1, 384, 1024, False), (1, 384, 1024, True),
                                         (3, 384, 1024, True), (5, 300, 256, False),
                                         (8, 4096, 11008, True), (70, 257, 512, False),
                                         (128, 256, 4096, True)])
def test_linear_bf16_bias(dev, orc, M, N, K, tiled):
    """A BFloat16 bias on a Q8_0 Linear (reference cuda_kernel_adapter.cpp:204-218:
    sgemm_nt, then add_bias of the widened bf16 in fp32): bit-identical to the same
    Linear with the widened fp32 bias on every path (GEMV, tiled GEMV, MFMA decode with
    split K, MFMA GEMM; raw and tiled weights), and within the path's bar of the oracle."""
    import torch
    note(f"bf16 bias M={M} N={N} K={K} tiled={tiled}")
    w, x = weight(160 + N, N, K), acts(161 + M, M, K)
    b32 = S.activations(162, (N,), tag=S.TAG_BIAS)
    b16 = (b32.view(np.uint32) >> 16).astype(np.uint16)        # bf16 bits (truncated)
    widened = (b16.astype(np.uint32) << 16).view(np.float32)    # exact widening
    dx, dw = to_dev(x, dev), to_dev(w, dev)
    if tiled:
        dwt = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
        capi.tile(dw, dwt, N, K)
        dw = dwt
    y16, y32 = empty_f32((M, N), dev), empty_f32((M, N), dev)
    capi.linear_bias_bf16(dx, dw, to_dev(b16, dev), y16, M, N, K, tiled=tiled)
    (capi.linear_tiled if tiled else capi.linear)(dx, dw, to_dev(widened, dev), y32, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y16, y32)
    err = rel_l2(to_host(y16), orc.linear(x, w, widened, M, N, K))
    assert err <= (MFMA_TOL if M >= 64 else GEMV_TOL), err


def test_linear_bf16_bias_errors(dev):
    FAKE = 0x1000
    code, msg = capi.linear_bias_bf16_status(FAKE, FAKE, FAKE + 1, FAKE, 1, 64, 64)
    assert code == 1 and "bias must be 2-byte aligned" in msg
    code, msg = capi.linear_bias_bf16_status(FAKE, FAKE, FAKE, FAKE, 1, 64, 48, tiled=True)
    assert code == 4 and "multiple of 32" in msg
