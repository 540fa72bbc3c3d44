"""C ABI checks that need no GPU: the library loads, exports exactly what the headers
declare, and rejects bad arguments before any HIP call (reference error conventions:
src/runtime/kernels/cuda_kernels.cu:53-130, :852-936, :1054-1073)."""
import glob
import os
import re
import subprocess

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
    assert lib.mle_q8_0_abi_version() == 4
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
    # MFMA decode: token tile 3 does not exist, 6 waves is not a shape, 65 splits too many
    for t in [(3, 4, 16, 0), (4, 6, 16, 0), (4, 4, 16, 1), (4, 4, 8, 0), (16, 4, 32, 0)]:
        rc = lib.mle_q8_0_linear_ex(FAKE, FAKE, None, FAKE, 1, 64, 64, 3, *t, None)
        assert rc == 1 and "MFMA decode shape" in capi.last_error(), t
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
