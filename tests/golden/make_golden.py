"""Write tests/golden/q8_0_golden.json from the reference's own CPU kernels.

Run in a container that has /root/reference:

    make -C oracle ref && python tests/golden/make_golden.py

The expected outputs come from oracle/_ref/libref_cpu_q8_0.so, i.e. the reference's
src/runtime/kernels/cpu_kernels.cpp compiled where it lies (oracle/Makefile); the inputs
come from llmengine_amd.synthetic (seeded, portable).  Only data is written: per case the
shape, the seeds, the SHA-256 of the fp32 output bytes and a set of sampled output bit
patterns (all of them for small outputs).  tests/test_oracle.py checks the C restatement
(oracle/q8_0_oracle.c) against these fixtures wherever the reference is absent.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from llmengine_amd import synthetic as S  # noqa: E402
import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q8_0_golden.json")

# (name, M, N, K, seed) for Linear; weights [N,K] with the benchmark's distributions.
LINEAR = [
    ("linear_1x64x256", 1, 64, 256, 101),
    ("linear_3x96x4096", 3, 96, 4096, 102),
    ("linear_8x16x11008", 8, 16, 11008, 103),
    ("linear_2x17x896", 2, 17, 896, 104),
    ("linear_c1_1x4096x4096", 1, 4096, 4096, 1),
    ("linear_c4_qkv_1x1152x896", 1, 1152, 896, 4),
    ("linear_c4_down_1x896x4864", 1, 896, 4864, 4),
]
# (name, M, N, K, seed) for MatMul; B [K,N] with blocks along N.
MATMUL = [
    ("matmul_2x32x32", 2, 32, 32, 201),
    ("matmul_3x64x160", 3, 64, 160, 202),
    ("matmul_5x256x512", 5, 256, 512, 203),
]
# (name, vocab, hidden, n_ids, seed)
EMBEDDING = [
    ("embedding_1000x896_300", 1000, 896, 300, 301),
    ("embedding_c5_151936x896_4096", 151936, 896, 4096, 5),
]
FULL_LIMIT = 512  # store every output value up to this many floats
N_SAMPLES = 64


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def samples(a: np.ndarray, seed: int):
    flat = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    if flat.size <= FULL_LIMIT:
        idx = np.arange(flat.size)
    else:
        rng = np.random.default_rng(seed)
        idx = np.unique(np.concatenate([[0, flat.size - 1],
                                        rng.integers(0, flat.size, N_SAMPLES)]))
    bits = flat.view(np.uint32)
    return [[int(i), f"{int(bits[i]):08x}"] for i in idx]


def linear_inputs(M, N, K, seed):
    w, _, _ = S.q8_0_weight(seed, N, K)
    x = S.activations(seed, (M, K))
    return x, w


def matmul_inputs(M, N, K, seed):
    b, _, _ = S.q8_0_weight(seed, K, N)
    a = S.activations(seed, (M, K))
    return a, b


def embedding_inputs(vocab, hidden, n_ids, seed):
    w, _, _ = S.q8_0_weight(seed, vocab, hidden)
    ids = S.token_ids(seed, n_ids, vocab)
    return w, ids


def known_answer_cases():
    """Inputs of the reference's own Q8_0 tests (integer quants, scale 1.0 or 0.5)."""
    cases = []
    # tests/test_cpu_kernels.cpp:138-168  (Linear M=2,N=3,K=32, scale 1.0)
    A = ((np.arange(64) % 7) - 3).astype(np.float32) * 0.25
    B = (((np.arange(96) * 5) % 17) - 8).astype(np.int8)
    cases.append(("known_linear_2x3x32_scale1", "linear", 2, 3, 32, A, B, 0x3C00))
    # tests/test_cuda_kernels.cpp:444-474  (Linear M=2,N=3,K=64, scale 0.5)
    A = ((np.arange(128) % 11) - 5).astype(np.float32) * 0.125
    B = (((np.arange(192) * 7) % 23) - 11).astype(np.int8)
    cases.append(("known_linear_2x3x64_scale05", "linear", 2, 3, 64, A, B, 0x3800))
    # tests/test_cpu_kernels.cpp:110-136  (MatMul M=2,K=2,N=32, scale 1.0)
    A = np.array([1.0, 2.0, -1.0, 3.0], dtype=np.float32)
    n = np.arange(32)
    B = np.concatenate([(n % 9) - 4, (n % 7) - 3]).astype(np.int8)
    cases.append(("known_matmul_2x32x2_scale1", "matmul", 2, 32, 2, A, B, 0x3C00))
    # tests/test_cuda_kernels.cpp:476-503  (MatMul M=2,N=64,K=32, scale 0.5)
    A = ((np.arange(64) % 13) - 6).astype(np.float32) * 0.125
    B = (((np.arange(2048) * 3) % 29) - 14).astype(np.int8)
    cases.append(("known_matmul_2x64x32_scale05", "matmul", 2, 64, 32, A, B, 0x3800))
    # tests/test_cpu_kernels.cpp:233-258  (Embedding vocab 3, hidden 32, ids {2,0})
    W = np.array([[r * 10 + h - 12 for h in range(32)] for r in range(3)], dtype=np.int8)
    cases.append(("known_embedding_3x32_ids20", "embedding", 3, 32, 0,
                  np.array([2, 0], np.int32), W.reshape(-1), 0x3C00))
    # tests/test_cuda_kernels.cpp:505-527  (Embedding vocab 3, hidden 64, ids {2,0,1}, 0.5)
    W = (((np.arange(192) * 5) % 31) - 15).astype(np.int8)
    cases.append(("known_embedding_3x64_ids201", "embedding", 3, 64, 0,
                  np.array([2, 0, 1], np.int32), W, 0x3800))
    return cases


def main():
    if not O.reference_available():
        sys.exit("oracle/_ref is not built: run `make -C oracle ref` where /root/reference exists")
    ref = O.reference()
    doc = {"generator": "tests/golden/make_golden.py",
           "expected_from": "reference src/runtime/kernels/cpu_kernels.cpp via oracle/_ref",
           "cases": []}

    for name, op, a1, a2, a3, A, Q, scale in known_answer_cases():
        packed = S.pack_q8_0_const_scale(Q, scale)
        if op == "linear":
            out = ref.sgemm_nt(A, packed, a1, a2, a3)
            entry = {"M": a1, "N": a2, "K": a3}
        elif op == "matmul":
            out = ref.sgemm(A, packed, a1, a2, a3)
            entry = {"M": a1, "N": a2, "K": a3}
        else:
            out = ref.embedding(packed, A, a2)
            entry = {"vocab": a1, "hidden": a2, "ids": A.tolist()}
        entry.update({"name": name, "op": op, "known_answer": True, "scale_bits": scale,
                      "activations": [float(v) for v in A] if op != "embedding" else None,
                      "quants": Q.astype(int).tolist(),
                      "sha256": digest(out), "samples": samples(out, 0)})
        doc["cases"].append(entry)

    for name, M, N, K, seed in LINEAR:
        x, w = linear_inputs(M, N, K, seed)
        out = ref.sgemm_nt(x, w, M, N, K)
        doc["cases"].append({"name": name, "op": "linear", "M": M, "N": N, "K": K,
                             "seed": seed, "sha256": digest(out), "samples": samples(out, seed)})
    for name, M, N, K, seed in MATMUL:
        a, b = matmul_inputs(M, N, K, seed)
        out = ref.sgemm(a, b, M, N, K)
        doc["cases"].append({"name": name, "op": "matmul", "M": M, "N": N, "K": K,
                             "seed": seed, "sha256": digest(out), "samples": samples(out, seed)})
    for name, vocab, hidden, n_ids, seed in EMBEDDING:
        w, ids = embedding_inputs(vocab, hidden, n_ids, seed)
        out = ref.embedding(w, ids, hidden)
        doc["cases"].append({"name": name, "op": "embedding", "vocab": vocab,
                             "hidden": hidden, "n_ids": n_ids, "seed": seed,
                             "sha256": digest(out), "samples": samples(out, seed)})

    # Exhaustive binary16 decode through the reference: a table whose block i has
    # scale bits i and first quant 1, gathered with ids 0..65535 -> out[i, 0] = d_i.
    q = np.zeros(65536 * 32, np.int8)
    q[0::32] = 1
    table = S.pack_q8_0(q, np.arange(65536, dtype=np.uint16).view(np.float16))
    dec = ref.embedding(table, np.arange(65536, dtype=np.int32), 32)[:, 0].copy()
    doc["f16_decode"] = {"sha256": digest(dec),
                         "nan_bits": sorted({f"{int(b):08x}" for b in
                                             dec.view(np.uint32)[np.isnan(dec)]})}

    with open(OUT, "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote", OUT, len(doc["cases"]), "cases")


if __name__ == "__main__":
    main()
