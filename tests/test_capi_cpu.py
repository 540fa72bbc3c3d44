"""C ABI checks that need no GPU: the library loads, exports exactly what the headers
declare, and rejects bad arguments before any HIP call (reference error conventions:
src/runtime/kernels/cuda_kernels.cu:53-130, :852-936, :1054-1073)."""
import glob
import os
import re
import subprocess

import numpy as np
import pytest

from llmengine_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x1000  # a non-null address that validation rejects before it is ever used


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(mle_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    assert lib.mle_q8_0_abi_version() == 7
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH],
                         stdout=subprocess.PIPE, text=True, check=True).stdout
    exported = set(re.findall(r" T (mle_\w+)", out))
    declared = declared_symbols()
    assert declared, "no declarations found in include/*.h"
    assert declared <= exported, declared - exported
    assert set(capi.EXPORTED) <= exported


def test_q8_0_bytes_rule():
    # ceil(numel/32)*34: cuda_kernel_adapter.cpp:86-97, gguf_parser.cpp:226-243
    assert capi.q8_0_bytes(0) == 0
    assert capi.q8_0_bytes(1) == 34
    assert capi.q8_0_bytes(32) == 34
    assert capi.q8_0_bytes(33) == 68
    assert capi.q8_0_bytes(4096 * 4096) == 4096 * 128 * 34
    assert capi.q8_0_bytes(-1) == 0


def test_linear_validation_errors():
    st = capi.linear_status
    code, msg = st(None, FAKE, None, FAKE, 1, 1, 32, stream=0)
    assert code == 1 and "A pointer must not be null" in msg
    code, msg = st(FAKE, None, None, FAKE, 1, 1, 32, stream=0)
    assert code == 1 and "B pointer" in msg
    code, msg = st(FAKE, FAKE, None, None, 1, 1, 32, stream=0)
    assert code == 1 and "C pointer" in msg
    for M, N, K, what in [(0, 1, 32, "M"), (1, 0, 32, "N"), (1, 1, 0, "K"), (-3, 1, 32, "M")]:
        code, msg = st(FAKE, FAKE, None, FAKE, M, N, K, stream=0)
        assert code == 1 and f"{what} must be positive" in msg
    code, msg = st(FAKE, FAKE, None, FAKE, 1, 2, 31, stream=0)
    assert code == 4 and "Q8_0" in msg and "32" in msg
    code, msg = st(FAKE + 4, FAKE, None, FAKE, 1, 2, 32, stream=0)
    assert code == 1 and "16-byte aligned" in msg
    code, msg = st(FAKE, FAKE + 1, None, FAKE, 1, 2, 32, stream=0)
    assert code == 1 and "aligned" in msg


def test_fused_linear_validation_errors():
    st = capi.linear_swiglu_status
    code, msg = st(FAKE, FAKE, None, FAKE, 1, 64, 64, stream=0)
    assert code == 1 and "up pointer must not be null" in msg
    code, msg = st(FAKE, None, FAKE, FAKE, 1, 64, 64, stream=0)
    assert code == 1 and "B pointer" in msg
    code, msg = st(FAKE, FAKE, FAKE, FAKE, 1, 64, 48, stream=0)
    assert code == 4 and "multiple of 32" in msg
    code, msg = st(FAKE, FAKE, FAKE + 1, FAKE, 1, 64, 64, stream=0)
    assert code == 1 and "up must be 2-byte aligned" in msg
    mt = capi.linear_multi_status
    for count in (0, 4):
        code, msg = mt(FAKE, [FAKE] * count, None, [FAKE] * count, [64] * count, 1, 64, stream=0)
        assert code == 1 and "count must be 1, 2 or 3" in msg
    code, msg = mt(FAKE, [FAKE, FAKE], None, [FAKE, FAKE], [64, 0], 1, 64, stream=0)
    assert code == 1 and "N must be positive" in msg
    code, msg = mt(FAKE, [FAKE, None], None, [FAKE, FAKE], [64, 64], 1, 64, stream=0)
    assert code == 1 and "B pointer" in msg
    code, msg = mt(FAKE, [FAKE], [FAKE + 2], [FAKE], [64], 1, 64, stream=0)
    assert code == 1 and "bias must be 4-byte aligned" in msg
    rc = capi.load().mle_q8_0_linear_multi(FAKE, 2, None, None, None, None, 1, 64, None)
    assert rc == 1 and "arrays must not be null" in capi.last_error()


def test_swiglu_validation_errors():
    st = capi.swiglu_status
    code, msg = st(None, FAKE, FAKE, 8, stream=0)
    assert code == 1 and "gate pointer" in msg
    code, msg = st(FAKE, FAKE, FAKE, -1, stream=0)
    assert code == 1 and "n must be >= 0" in msg
    code, msg = st(FAKE, FAKE + 2, FAKE, 8, stream=0)
    assert code == 1 and "up must be 4-byte aligned" in msg


def test_matmul_workspace_size():
    """MLE_OP_MATMUL: decode-size MatMuls spread K over workgroups and need
    workspace: up to 8 rows of A, a partial tile of 256 columns x the token tile per
    workgroup plus a counter per tile (16 tiles x 16 splits at 1 x 4096 x 4096);
    9-63 rows, [S][M][N] partial floats; wide N at small M needs none; from 64 rows
    of A the MatMul runs the bf16 MFMA GEMM, which needs its bf16 copy of A (rows
    rounded up to 32, K to 64) plus any split-K partials and counters."""
    b, c = capi.workspace_size(capi.OP_MATMUL, 1, [4096], 4096)
    assert b >= 16 * 16 * 256 * 4 and c >= 16
    b, c = capi.workspace_size(capi.OP_MATMUL, 16, [4096], 4096)
    assert b >= 16 * 4096 * 4 and c == 0
    assert capi.workspace_size(capi.OP_MATMUL, 63, [512], 256) == (0, 0)
    assert capi.workspace_size(capi.OP_MATMUL, 1, [151936], 896) == (0, 0)
    b, c = capi.workspace_size(capi.OP_MATMUL, 512, [4096], 4096)
    assert b >= 512 * 4096 * 2
    b, c = capi.workspace_size(capi.OP_MATMUL, 77, [1056], 1312)
    assert b >= 96 * 1344 * 2
    code, msg, _, _ = capi.workspace_size_status(capi.OP_MATMUL, 1, [48], 64)
    assert code == 4 and "multiple of 32" in msg
    code, msg, _, _ = capi.workspace_size_status(capi.OP_MATMUL, 1, [64, 64], 64)
    assert code == 1 and "count 1" in msg


def test_swiglu_workspace_follows_the_decode_kernel():
    """MLE_OP_LINEAR_SWIGLU: the gate/up pair (tiled or raw) at 3-4 and 6-8 tokens on
    512-1024 row groups per weight runs the row-range decode (no workspace); 5 tokens
    and 256-group weights run the split-K decode (partials and counters)."""
    N, K = 11008, 4096
    for M in (3, 4, 6, 8):
        for tiled in (True, False):
            assert capi.workspace_size(capi.OP_LINEAR_SWIGLU, M, [N, N], K, tiled) == (0, 0), M
    for M, n, tiled in ((5, N, True), (5, N, False), (4, 4096, True), (8, 4096, False)):
        b, c = capi.workspace_size(capi.OP_LINEAR_SWIGLU, M, [n, n], K, tiled)
        assert b > 0 and c > 0, (M, n, tiled)


def test_probe_stream_read_validation_errors():
    st = capi.probe_stream_read_status
    code, msg = st(None, 64, FAKE, stream=0)
    assert code == 1 and "src pointer" in msg
    code, msg = st(FAKE, 64, None, stream=0)
    assert code == 1 and "sink pointer" in msg
    code, msg = st(FAKE, 40, FAKE, stream=0)
    assert code == 1 and "multiple of 16" in msg
    code, msg = st(FAKE, -16, FAKE, stream=0)
    assert code == 1 and "multiple of 16" in msg
    code, msg = st(FAKE + 8, 64, FAKE, stream=0)
    assert code == 1 and "src must be 16-byte aligned" in msg


def test_top_tokens_validation_errors():
    st = capi.top_tokens_status
    code, msg = st(None, 1, 10, 5, FAKE, FAKE, stream=0)
    assert code == 1 and "logits pointer" in msg
    code, msg = st(FAKE, 1, 10, 5, None, FAKE, stream=0)
    assert code == 1 and "ids pointer" in msg
    code, msg = st(FAKE, 1, 10, 5, FAKE, None, stream=0)
    assert code == 1 and "probs pointer" in msg
    code, msg = st(FAKE, 0, 10, 5, FAKE, FAKE, stream=0)
    assert code == 1 and "rows must be positive" in msg
    code, msg = st(FAKE, 1, 0, 5, FAKE, FAKE, stream=0)
    assert code == 1 and "n must be positive" in msg
    # top_n <= 0: the reference returns an empty list; nothing is launched
    assert st(FAKE, 1, 10, 0, FAKE, FAKE, stream=0)[0] == 0
    assert st(FAKE, 1, 10, -3, FAKE, FAKE, stream=0)[0] == 0
    code, msg = st(FAKE, 70000, 10, 5, FAKE, FAKE, stream=0)
    assert code == 4 and "65535" in msg
    code, msg = st(FAKE, 1, 1000, 129, FAKE, FAKE, stream=0)
    assert code == 4 and "at most 128" in msg
    # candidates of a row must fit one workgroup: n <= (16384 / k) * 2048
    code, msg = st(FAKE, 1, 262145, 128, FAKE, FAKE, stream=0)
    assert code == 4 and "at most 262144" in msg
    code, msg = st(FAKE + 2, 1, 10, 5, FAKE, FAKE, stream=0)
    assert code == 1 and "logits must be 4-byte aligned" in msg


def test_argmax_validation_errors():
    st = capi.argmax_status
    code, msg = st(None, 1, 10, FAKE, stream=0)
    assert code == 1 and "logits pointer" in msg
    code, msg = st(FAKE, 1, 10, None, stream=0)
    assert code == 1 and "idx pointer" in msg
    code, msg = st(FAKE, 0, 10, FAKE, stream=0)
    assert code == 1 and "rows must be positive" in msg
    code, msg = st(FAKE, 1, 0, FAKE, stream=0)
    assert code == 1 and "n must be positive" in msg
    code, msg = st(FAKE, 70000, 10, FAKE, stream=0)
    assert code == 4 and "65535" in msg
    code, msg = st(FAKE + 2, 1, 10, FAKE, stream=0)
    assert code == 1 and "logits must be 4-byte aligned" in msg


def test_linear_ex_rejects_bad_launch_shape():
    lib = capi.load()
    rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 1, 3, 32, 1, 0, None)
    assert rc == 1 and "launch shape" in capi.last_error()
    rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 5, 0, 0, 0, 0, None)
    assert rc == 1 and "path" in capi.last_error()
    # row-span GEMV (t3 = rows per workgroup): 4 rows and a one-token tile only
    for t in [(1, 64, 1, 8), (2, 64, 1, 4), (1, 64, 1, 16), (1, 64, 1, -4)]:
        rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 1, *t, None)
        assert rc == 1 and "GEMV launch shape" in capi.last_error(), t
    # MFMA decode: token tile 3 does not exist, 6 waves is not a shape, 8-block slices
    # and 16-token 32-block slices do not exist
    for t in [(3, 4, 16, 0), (4, 6, 16, 0), (4, 4, 8, 0), (16, 4, 32, 0)]:
        rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 3, *t, None)
        assert rc == 1 and "MFMA decode shape" in capi.last_error(), t
    # hybrid MFMA decode shapes (t3 = 1..4): a 4- or 8-token tile only
    for t in [(2, 4, 16, 1), (16, 4, 16, 4)]:
        rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 3, *t, None)
        assert rc == 1 and "hybrid MFMA decode shape" in capi.last_error(), t
    fake16 = FAKE + 64 - FAKE % 64  # 16-byte aligned, never dereferenced
    for t in [(2, 4, 16, 1), (4, 4, 16, 5), (8, 4, 16, -1)]:
        rc = lib.mle_q8_0_linear_tiled_ex(FAKE, fake16, None, FAKE, 1, 64, 64, 3, *t, None)
        assert rc == 1 and "MFMA decode shape" in capi.last_error(), t
    rc = lib.mle_q8_0_linear_tiled_ex(FAKE, fake16, None, FAKE, 1, 64, 64, 2, 0, 0, 0, 0, None)
    assert rc == 1 and "path on tiled weights" in capi.last_error()
    # MFMA GEMM: t3 unused, 65 splits too many, 1 / 192 tile rows, 80 tile columns,
    # 256 x 128 tiles
    for t in [(0, 0, 0, 1), (65, 0, 0, 0), (2, 1, 0, 0), (0, 192, 0, 0), (1, 128, 80, 0),
              (1, 256, 128, 0)]:
        rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 2, *t, None)
        assert rc == 1 and "MFMA GEMM shape" in capi.last_error(), t


def test_matmul_validation_errors():
    st = capi.matmul_status
    code, msg = st(FAKE, FAKE, None, 1, 32, 32, stream=0)
    assert code == 1 and "C pointer" in msg
    code, msg = st(FAKE, FAKE, FAKE, 1, 32, 31, stream=0)
    assert code == 4 and "multiples of 32" in msg
    code, msg = st(FAKE, FAKE, FAKE, 1, 33, 32, stream=0)
    assert code == 4 and "multiples of 32" in msg
    code, msg = st(FAKE, FAKE, FAKE, 1, 32, -32, stream=0)
    assert code == 1 and "K must be positive" in msg


def test_embedding_validation_errors():
    st = capi.embedding_status
    code, msg = st(FAKE, None, FAKE, 1, 10, 32, stream=0)
    assert code == 1 and "ids pointer" in msg
    code, msg = st(FAKE, FAKE, FAKE, -1, 10, 32, stream=0)
    assert code == 1 and "seq_len" in msg
    code, msg = st(FAKE, FAKE, FAKE, 1, 0, 32, stream=0)
    assert code == 1 and "vocab_size must be positive" in msg
    code, msg = st(FAKE, FAKE, FAKE, 1, 10, 48, stream=0)
    assert code == 4 and "multiple of 32" in msg
    # empty input is a no-op, as on the reference CPU path (cpu_kernel_adapter.cpp:67-70)
    code, msg = st(FAKE, FAKE, FAKE, 0, 10, 32, stream=0)
    assert code == 0 and msg == ""


def test_last_error_is_cleared_by_success():
    capi.embedding_status(FAKE, None, FAKE, 1, 10, 32, stream=0)
    assert capi.last_error() != ""
    capi.embedding_status(FAKE, FAKE, FAKE, 0, 10, 32, stream=0)
    assert capi.last_error() == ""


def test_product_package_does_not_import_oracle():
    pkg = os.path.join(ROOT, "llmengine_amd")
    for path in glob.glob(os.path.join(pkg, "**", "*.*"), recursive=True):
        if path.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
            text = open(path).read()
            assert not re.search(r"^\s*(import|from)\s+oracle\b", text, re.M), path
            assert "q8_0_oracle" not in text and "liboracle" not in text, path


def test_tiled_bytes_rule():
    # G*KP*1088 with G = ceil(N/16) row groups and KP = ceil(K/64) block pairs
    assert capi.tiled_bytes(4096, 11008) == 4096 * 344 * 34  # no padding
    assert capi.tiled_bytes(17, 96) == 2 * 2 * 1088          # rows and a block padded
    assert capi.tiled_bytes(1, 32) == 1088
    assert capi.tiled_bytes(151936, 896) == 151936 * 28 * 34
    for bad in [(0, 32), (16, 0), (16, 48), (-1, 32)]:
        assert capi.tiled_bytes(*bad) == 0


@pytest.mark.parametrize("N,K", [(1, 32), (17, 96), (33, 4128), (100, 992)])
def test_tile_reference_layout(N, K):
    """The numpy tiler that checks the device repack: a permutation of the raw
    bytes plus zero padding (round trip), and each slot where the layout puts it
    (explicit loops over the formula of include/mle_q8_0.h)."""
    from helpers import tile_ref, tiled_shape, untile_ref
    from llmengine_amd import synthetic as S
    raw = S.q8_0_weight(5 + N, N, K)[0]
    t = tile_ref(raw, N, K)
    assert t.size == capi.tiled_bytes(N, K)
    assert np.array_equal(untile_ref(t, N, K), raw)
    KB, KP, G = tiled_shape(N, K)
    blk = raw.reshape(N, KB, 34)
    zero8, zero2 = np.zeros(8, np.uint8), np.zeros(2, np.uint8)
    for g in range(G):
        for p in range(KP):
            for l in range(64):
                sub, r = l // 16, l % 16
                for h in range(2):
                    row, b = 16 * g + r, 2 * p + h
                    want = blk[row, b, 2 + 8 * sub:10 + 8 * sub] if row < N and b < KB else zero8
                    off = (g * KP + p) * 1024 + 16 * l + 8 * h
                    assert np.array_equal(t[off:off + 8], want), (g, p, l, h)
            for r in range(16):
                for h in range(2):
                    row, b = 16 * g + r, 2 * p + h
                    want = blk[row, b, 0:2] if row < N and b < KB else zero2
                    off = G * KP * 1024 + (g * KP + p) * 64 + 4 * r + 2 * h
                    assert np.array_equal(t[off:off + 2], want), (g, p, r, h)
    # a dropped or duplicated slot would break the round trip; a swapped pair of
    # halves would break the loop check
    bad = t.copy()
    bad[8:16], bad[0:8] = t[0:8], t[8:16]
    if not np.array_equal(t[0:8], t[8:16]):
        assert not np.array_equal(untile_ref(bad, N, K), raw)


def test_tile_validation_errors():
    st = capi.tile_status
    code, msg = st(None, FAKE, 16, 32, stream=0)
    assert code == 1 and "w_q8_0 pointer" in msg
    code, msg = st(FAKE, None, 16, 32, stream=0)
    assert code == 1 and "w_tiled pointer" in msg
    code, msg = st(FAKE, FAKE + 0x100000, 0, 32, stream=0)
    assert code == 1 and "N must be positive" in msg
    code, msg = st(FAKE, FAKE + 0x100000, 16, 48, stream=0)
    assert code == 4 and "multiple of 32" in msg
    code, msg = st(FAKE + 1, FAKE + 0x100000, 16, 32, stream=0)
    assert code == 1 and "2-byte aligned" in msg
    code, msg = st(FAKE, FAKE + 0x100008, 16, 32, stream=0)
    assert code == 1 and "16-byte aligned" in msg
    # 16 rows x 1 block: raw [FAKE, FAKE + 544), tiled 1088 bytes
    code, msg = st(FAKE, FAKE + 512, 16, 32, stream=0)
    assert code == 1 and "overlap" in msg
    code, msg = capi.linear_tiled_status(FAKE, FAKE + 2, None, FAKE, 1, 16, 32, stream=0)
    assert code == 1 and "16-byte aligned" in msg
    code, msg = capi.linear_tiled_status(FAKE, FAKE, None, FAKE, 1, 16, 48, stream=0)
    assert code == 4 and "multiple of 32" in msg
    code, msg = capi.linear_swiglu_tiled_status(FAKE, FAKE, FAKE + 2, FAKE, 1, 16, 32, stream=0)
    assert code == 1 and "16-byte aligned" in msg
    code, msg = capi.linear_multi_status(FAKE, [FAKE, FAKE + 4], None, [FAKE, FAKE], [16, 16],
                                         1, 32, stream=0, tiled=True)
    assert code == 1 and "16-byte aligned" in msg


def test_workspace_growth_rule():
    """Capacities never shrink; a buffer that grows takes max(capacity, need, minimum),
    so alternating a counter-heavy and a partial-heavy need settles after one pair."""
    MIN_B, MIN_C = 4 << 20, 4096
    assert capi.workspace_plan_growth(0, 0, 100, 10) == (True, MIN_B, MIN_C)
    assert capi.workspace_plan_growth(MIN_B, MIN_C, MIN_B, MIN_C) == (False, MIN_B, MIN_C)
    # more counters only: the partial buffer keeps its (larger) capacity
    assert capi.workspace_plan_growth(64 << 20, MIN_C, 1 << 20, 20000) == (True, 64 << 20, 20000)
    # more bytes only: the counter buffer keeps its capacity
    assert capi.workspace_plan_growth(MIN_B, 20000, 8 << 20, 10) == (True, 8 << 20, 20000)
    caps, grows = (0, 0), 0
    for need in [(8 << 20, 100), (1 << 20, 50000)] * 3:
        grow, b, c = capi.workspace_plan_growth(*caps, *need)
        grows += grow
        caps = (b, c)
    assert grows == 2 and caps == (8 << 20, 50000)
    # a buffer that must grow at least doubles, so retained old buffers stay bounded
    assert capi.workspace_plan_growth(8 << 20, MIN_C, 9 << 20, 10) == (True, 16 << 20, MIN_C)
    assert capi.workspace_plan_growth(8 << 20, MIN_C, 40 << 20, 3 * MIN_C) == (
        True, 40 << 20, 3 * MIN_C)


def test_workspace_size_matches_launch_plan():
    """mle_q8_0_workspace_size runs the path choice of the Linear calls without launching
    (no GPU needed): decode launches with K split need partials and 128-byte counters;
    the FP32 GEMV and the tiled GEMV need nothing; prefill needs the bf16 copy of X."""
    ws = capi.workspace_size
    assert ws(capi.OP_LINEAR, 1, [4096], 4096) == (0, 0)              # FP32 GEMV
    assert ws(capi.OP_LINEAR, 1, [4096], 4096, tiled=True) == (0, 0)  # tiled GEMV
    b, c = ws(capi.OP_LINEAR, 16, [4096], 11008)                      # MFMA decode, 22 splits
    # every row x 22 K slices x 16 tokens of partial floats; 32 counters per row tile
    # (4-wave tiles of 64 rows; o_proj's 4096-element rows take 8-wave tiles of 128
    # rows when tiled)
    assert b == 4096 * 22 * 16 * 4 and c == (4096 // 64) * 32
    # 6-8 tokens, raw or tiled, the hybrid decode: every row x 8 splits of 44 blocks x
    # 8 tokens, one counter line per 4-group (64-row) workgroup column
    for tiled in (False, True):
        assert ws(capi.OP_LINEAR, 8, [4096], 11008, tiled=tiled) == (4096 * 8 * 8 * 4,
                                                                     (4096 // 64) * 32)
    bo, co = ws(capi.OP_LINEAR, 8, [4096], 4096, tiled=True)         # o_proj: 8 splits
    assert bo == 4096 * 8 * 8 * 4 and co == (4096 // 128) * 32
    bg, cg = ws(capi.OP_LINEAR, 512, [11008], 4096)                   # prefill GEMM
    assert bg >= 512 * 4096 * 2                                       # bf16 copy of X
    b3, c3 = ws(capi.OP_LINEAR_MULTI, 8, [4096, 4096, 4096], 4096)
    b1, c1 = ws(capi.OP_LINEAR, 8, [12288], 4096)
    assert b3 > 0 and c3 > 0 and b1 > 0
    bs, cs = ws(capi.OP_LINEAR_SWIGLU, 5, [11008, 11008], 4096)     # split-K SwiGLU
    assert bs > 0 and cs > 0
    assert ws(capi.OP_LINEAR_SWIGLU, 4, [11008, 11008], 4096) == (0, 0)  # row-range SwiGLU
    # chunks of 16 tokens share one workspace: the need is the largest chunk's
    assert ws(capi.OP_LINEAR, 40, [4096], 11008) == ws(capi.OP_LINEAR, 16, [4096], 11008)
    code, msg, _, _ = capi.workspace_size_status(capi.OP_LINEAR, 1, [64], 48)
    assert code == 4 and "multiple of 32" in msg
    code, msg, _, _ = capi.workspace_size_status(capi.OP_LINEAR_SWIGLU, 1, [64, 32], 64)
    assert code == 1 and "equal N" in msg
    code, msg, _, _ = capi.workspace_size_status(7, 1, [64], 64)
    assert code == 1 and "unknown op" in msg
