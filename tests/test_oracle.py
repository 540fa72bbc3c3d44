"""Pins the CPU oracle (oracle/q8_0_oracle.c) before anything is checked against it.

Each function of the oracle is pinned by checks chosen so that a plausible mistake (a
dropped term, a wrong sign or index, a transposed operand, a different rounding order)
fails at least one of them:

* exhaustive binary16 decode against numpy.float16 (closed form) and against the
  reference's own decode (golden SHA-256 of all 65536 patterns);
* the reference's known-answer tests (integer quants x dyadic activations, scale 1 or
  1/2: every partial sum is exact, so any order gives the same bits) against exact
  float64 arithmetic;
* the golden fixtures produced by the reference's compiled cpu_kernels.cpp
  (tests/golden/make_golden.py), bit for bit;
* the reference build itself (oracle/_ref) where it exists here, bit for bit;
* an FP64 brute force with a relative-L2 bound, plus mutation checks showing that
  the bound rejects the plausible mistakes listed above.
"""
import hashlib

import numpy as np
import pytest

from llmengine_amd import synthetic as S
import oracle as O


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rel_l2(a, ref):
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(a - ref) / np.linalg.norm(ref))


# ---------------------------------------------------------------- binary16 decode

def test_f16_decode_exhaustive_closed_form(orc):
    table = orc.f16_table()
    all_bits = np.arange(65536, dtype=np.uint16)
    npy = all_bits.view(np.float16).astype(np.float32)
    finite_or_inf = ~np.isnan(npy)
    assert np.array_equal(bits(table)[finite_or_inf], bits(npy)[finite_or_inf])
    # NaNs: default quiet NaN carrying the input sign (cpu_kernels.cpp:29-31).
    nan_idx = np.nonzero(~finite_or_inf)[0]
    assert nan_idx.size == 2046
    expect = np.where(all_bits[nan_idx] & 0x8000, 0xFFC00000, 0x7FC00000).astype(np.uint32)
    assert np.array_equal(bits(table)[nan_idx], expect)
    # Spot values, including every subnormal boundary.
    assert orc.f16_to_f32(0x0001) == 2.0 ** -24
    assert orc.f16_to_f32(0x03FF) == 1023 * 2.0 ** -24
    assert orc.f16_to_f32(0x0400) == 2.0 ** -14
    assert orc.f16_to_f32(0x7BFF) == 65504.0
    assert np.signbit(orc.f16_to_f32(0x8000)) and orc.f16_to_f32(0x8000) == 0.0


def test_f16_decode_matches_reference_golden(orc, golden):
    table = orc.f16_table()
    assert sha(table) == golden["f16_decode"]["sha256"]


# ---------------------------------------------------------------- known answers

def _known(golden):
    return [c for c in golden["cases"] if c.get("known_answer")]


def test_known_answer_cases_exact(orc, golden):
    cases = _known(golden)
    assert len(cases) == 6
    for c in cases:
        Q = np.array(c["quants"], dtype=np.int8)
        packed = S.pack_q8_0_const_scale(Q, c["scale_bits"])
        scale = float(np.array([c["scale_bits"]], np.uint16).view(np.float16)[0])
        if c["op"] == "linear":
            M, N, K = c["M"], c["N"], c["K"]
            A = np.array(c["activations"], np.float32)
            out = orc.sgemm_nt(A, packed, M, N, K)
            exact = A.reshape(M, K).astype(np.float64) @ (
                Q.reshape(N, K).astype(np.float64).T * scale)
        elif c["op"] == "matmul":
            M, N, K = c["M"], c["N"], c["K"]
            A = np.array(c["activations"], np.float32)
            out = orc.sgemm(A, packed, M, N, K)
            exact = A.reshape(M, K).astype(np.float64) @ (
                Q.reshape(K, N).astype(np.float64) * scale)
        else:
            ids = np.array(c["ids"], np.int32)
            out = orc.embedding(packed, ids, c["hidden"])
            exact = Q.reshape(c["vocab"], c["hidden"]).astype(np.float64)[ids] * scale
        assert np.array_equal(bits(out), bits(exact.astype(np.float32))), c["name"]
        assert sha(out) == c["sha256"], c["name"]


# ---------------------------------------------------------------- golden fixtures

def _run_case(orc, c):
    if c["op"] == "linear":
        w, _, _ = S.q8_0_weight(c["seed"], c["N"], c["K"])
        x = S.activations(c["seed"], (c["M"], c["K"]))
        return orc.sgemm_nt(x, w, c["M"], c["N"], c["K"])
    if c["op"] == "matmul":
        b, _, _ = S.q8_0_weight(c["seed"], c["K"], c["N"])
        a = S.activations(c["seed"], (c["M"], c["K"]))
        return orc.sgemm(a, b, c["M"], c["N"], c["K"])
    w, _, _ = S.q8_0_weight(c["seed"], c["vocab"], c["hidden"])
    ids = S.token_ids(c["seed"], c["n_ids"], c["vocab"])
    return orc.embedding(w, ids, c["hidden"])


@pytest.mark.parametrize("name", [
    "linear_1x64x256", "linear_3x96x4096", "linear_8x16x11008", "linear_2x17x896",
    "linear_c1_1x4096x4096", "linear_c4_qkv_1x1152x896", "linear_c4_down_1x896x4864",
    "matmul_2x32x32", "matmul_3x64x160", "matmul_5x256x512",
    "embedding_1000x896_300", "embedding_c5_151936x896_4096"])
def test_oracle_matches_reference_golden(orc, golden, name):
    c = next(c for c in golden["cases"] if c["name"] == name)
    out = _run_case(orc, c)
    flat = bits(out).reshape(-1)
    for idx, hexbits in c["samples"]:
        assert int(flat[idx]) == int(hexbits, 16), (name, idx)
    assert sha(out) == c["sha256"], name


# ---------------------------------------------------------------- reference build

needs_ref = pytest.mark.skipif(not O.reference_available(),
                               reason="oracle/_ref (reference build) not present")


@needs_ref
@pytest.mark.parametrize("M,N,K", [(1, 1, 32), (3, 17, 96), (2, 40, 4096), (5, 33, 896)])
def test_linear_bitexact_vs_reference_build(orc, M, N, K):
    ref = O.reference()
    w, _, _ = S.q8_0_weight(7 + M + N, N, K)
    x = S.activations(9 + K, (M, K))
    assert np.array_equal(bits(orc.sgemm_nt(x, w, M, N, K)), bits(ref.sgemm_nt(x, w, M, N, K)))


@needs_ref
@pytest.mark.parametrize("M,N,K", [(1, 32, 1), (3, 96, 64), (4, 64, 1000)])
def test_matmul_bitexact_vs_reference_build(orc, M, N, K):
    ref = O.reference()
    b, _, _ = S.q8_0_weight(11 + N, K, N)
    a = S.activations(13 + K, (M, K))
    assert np.array_equal(bits(orc.sgemm(a, b, M, N, K)), bits(ref.sgemm(a, b, M, N, K)))


@needs_ref
def test_embedding_and_special_scales_vs_reference_build(orc):
    ref = O.reference()
    # every binary16 class as a scale: zeros, subnormals, normals, max, Inf, NaN
    specials = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0x7BFF,
                         0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE00], np.uint16)
    q = S.quants(21, specials.size * 32)
    table = S.pack_q8_0(q, specials.view(np.float16))
    ids = np.arange(specials.size, dtype=np.int32)[::-1].copy()
    a = orc.embedding(table, ids, 32)
    b = ref.embedding(table, ids, 32)
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(bits(a)[~nan], bits(b)[~nan])


# ---------------------------------------------------------------- FP64 brute force

@pytest.mark.parametrize("M,N,K", [(1, 256, 4096), (8, 64, 11008), (4, 96, 896)])
def test_linear_fp64_bound(orc, M, N, K):
    w, _, _ = S.q8_0_weight(31, N, K)
    x = S.activations(32, (M, K))
    Wd = S.dequantize(w, N * K).reshape(N, K)
    ref64 = x.astype(np.float64) @ Wd.T
    assert rel_l2(orc.sgemm_nt(x, w, M, N, K), ref64) < 5e-6


def test_matmul_fp64_bound(orc):
    M, N, K = 3, 256, 2048
    b, _, _ = S.q8_0_weight(33, K, N)
    a = S.activations(34, (M, K))
    ref64 = a.astype(np.float64) @ S.dequantize(b, K * N).reshape(K, N)
    assert rel_l2(orc.sgemm(a, b, M, N, K), ref64) < 5e-6


def test_embedding_closed_form(orc):
    vocab, hidden = 500, 96
    w, q, d = S.q8_0_weight(35, vocab, hidden)
    ids = S.token_ids(36, 257, vocab)
    # closed form: fp32(d) * fp32(q), one rounding (the product is exact in fp64)
    dq = (d.astype(np.float32).reshape(-1, 1) * q.reshape(-1, 32).astype(np.float32))
    expect = dq.reshape(vocab, hidden)[ids]
    out = orc.embedding(w, ids, hidden)
    assert np.array_equal(bits(out), bits(expect))


def test_dequantize_closed_form_and_embedding(orc):
    """Whole-stream dequantisation: the closed form fp32(d) * fp32(q) (numpy float16
    decode, one rounding) bit for bit, including a partial last block and every class
    of binary16 scale (subnormal, zero, inf, NaN by position); and the same bits as
    the embedding gather of every row."""
    vocab, hidden = 300, 64
    w, q, d = S.q8_0_weight(38, vocab, hidden)
    dq = (d.astype(np.float32).reshape(-1, 1) * q.reshape(-1, 32).astype(np.float32)).reshape(-1)
    for n in (vocab * hidden, vocab * hidden - 5, 33, 1):
        out = orc.dequantize_q8_0(w, n)
        assert np.array_equal(bits(out), bits(dq[:n])), n
    rows = orc.embedding(w, np.arange(vocab, dtype=np.int32), hidden)
    assert np.array_equal(bits(orc.dequantize_q8_0(w, vocab * hidden)), bits(rows.reshape(-1)))
    special = np.array([0x0001, 0x03ff, 0x0000, 0x8000, 0x7c00, 0xfc00, 0x7e00, 0x3c00],
                       dtype=np.uint16)
    ws = w[: 8 * 34].copy()
    ws.reshape(8, 34)[:, :2] = special.view(np.uint8).reshape(8, 2)
    got = orc.dequantize_q8_0(ws, 8 * 32)
    want = (special.view(np.float16).astype(np.float32).reshape(-1, 1)
            * ws.reshape(8, 34)[:, 2:].view(np.int8).astype(np.float32)).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(bits(got[fin]), bits(want[fin]))


def test_embedding_zero_fill_semantics(orc):
    vocab, hidden = 40, 64
    w, _, _ = S.q8_0_weight(37, vocab, hidden)
    ids = np.array([3, -1, 39, 40, 7, 2 ** 31 - 1, -2 ** 31], np.int32)
    out = orc.embedding_zero_fill(w, ids, vocab, hidden)
    valid = (ids >= 0) & (ids < vocab)
    ref = orc.embedding(w, np.where(valid, ids, 0).astype(np.int32), hidden)
    assert np.array_equal(bits(out[valid]), bits(ref[valid]))
    assert np.all(bits(out[~valid]) == 0)


def test_linear_bias_epilogue(orc):
    M, N, K = 3, 48, 256
    w, _, _ = S.q8_0_weight(38, N, K)
    x = S.activations(39, (M, K))
    bias = S.activations(40, (N,), tag=S.TAG_BIAS)
    out = orc.linear(x, w, bias, M, N, K)
    base = orc.sgemm_nt(x, w, M, N, K)
    assert np.array_equal(bits(out), bits(base + bias[None, :]))


# ---------------------------------------------------------------- mutation checks

def test_fp64_bound_rejects_plausible_mistakes():
    """Each deliberately wrong dequantisation below must break the 5e-6 bound."""
    M, N, K = 2, 64, 1024
    w, q, d = S.q8_0_weight(41, N, K)
    x = S.activations(42, (M, K)).astype(np.float64)
    good = S.dequantize(w, N * K).reshape(N, K)
    ref = x @ good.T
    qf = q.astype(np.float64).reshape(N, K)
    df = d.astype(np.float64).reshape(N, K // 32)
    mutants = {
        "transposed_rows": x @ np.ascontiguousarray(good.reshape(K, N)),
        "dropped_last_block": x @ np.concatenate(
            [good[:, :-32], np.zeros((N, 32))], axis=1).T,
        "negated_scale": x @ (-good).T,
        "scale_of_next_block": x @ (qf * np.repeat(np.roll(df, -1, axis=1), 32, axis=1)).T,
        "quant_index_off_by_one": x @ (np.roll(qf, 1, axis=1) * np.repeat(df, 32, axis=1)).T,
        "unsigned_quants": x @ ((qf % 256) * np.repeat(df, 32, axis=1)).T,
        "bf16_rounded_weights": x @ good.astype(np.float32).view(np.uint32).__and__(
            0xFFFF0000).view(np.float32).astype(np.float64).T,
    }
    for name, bad in mutants.items():
        assert rel_l2(bad, ref) > 1e-4, name


# ---------------------------------------------------------------- generator

def test_synthetic_distributions_and_slicing():
    d = S.scales_f16(7, 1 << 18)
    b = d.view(np.uint16)
    sub = np.mean(((b >> 10) & 31) == 0)
    assert 0.29 < sub < 0.315  # ~30.2 % of scales are binary16 subnormals
    q = S.quants(7, 1 << 20)
    assert q.min() == -127 and q.max() == 127
    x = S.activations(7, (1 << 18,))
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    # counter-based: any slice regenerates bit-identically
    full = S.u64_stream(9, 2, 0, 1000)
    assert np.array_equal(full[400:700], S.u64_stream(9, 2, 400, 300))
    assert np.array_equal(S.normals64(9, 1, 0, 50)[10:20], S.normals64(9, 1, 10, 10))
    ids = S.token_ids(5, 4096, 151936)
    assert ids.min() >= 0 and ids.max() < 151936
