"""The no-allocation Linear entry point (mle_q8_0_linear_noalloc) against mle_q8_0_linear.

The variant keeps its split-K partials, tile counters and prefill scratch in the
library's static device array instead of the per-stream workspace.  Bar: the same
kernels run on the same operands, so outputs are bit-identical to mle_q8_0_linear (the
Linear paths themselves are held to the oracle by the other GPU tests).  Each pair of
calls runs twice in a row on the shared array, the second call with a smaller input, so
stale partials or counters left by the first call would show; a chain of calls with K splits of
different shapes is also enqueued back to back with a single synchronisation at the end
(calls ordered on one stream share the array safely).  A child process checks the
array's first use under graph capture (refused) and a captured call with K splits (the
hybrid decode) replayed
between eager calls.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

from helpers import empty_f32, note, to_dev
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _operands(dev, seed, M, N, K, bias):
    w, _, _ = S.q8_0_weight(seed, N, K)
    x = S.activations(seed + 1, (M, K))
    b = S.activations(seed + 2, (N,), tag=S.TAG_BIAS) if bias else None
    return to_dev(x, dev), to_dev(w, dev), (to_dev(b, dev) if bias else None)


@pytest.mark.parametrize("first,second", [
    ((8, 4096, 11008, False), (4, 1024, 4096, True)),      # hybrid, then split-K: 8 splits each
    ((512, 4096, 11008, False), (96, 512, 2048, True)),    # prefill GEMM: 28 MB of scratch
    ((16, 2048, 8192, True), (5, 1024, 4096, False)),      # split-K decode, other tile/splits
])
def test_noalloc_matches_linear_two_calls(dev, first, second):
    import torch
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        before = capi.workspace_info(stream)
        for i, (M, N, K, bias) in enumerate((first, second)):
            note(f"linear_noalloc call {i + 1}: M={M} N={N} K={K} bias={bias}")
            dx, dw, db = _operands(dev, 200 + 10 * i, M, N, K, bias)
            y0, y1 = empty_f32((M, N), dev), empty_f32((M, N), dev)
            capi.linear_noalloc(dx, dw, db, y0, M, N, K, stream=stream)
            capi.linear(dx, dw, db, y1, M, N, K, stream=torch.cuda.Stream())
            torch.cuda.synchronize()
            assert torch.isfinite(y0).all()
            assert torch.equal(y0, y1), (M, N, K)
        # the no-allocation calls never created this stream's workspace
        assert capi.workspace_info(stream) == before == (0, 0, 0)


def test_noalloc_rejects_shapes_beyond_its_scratch(dev):
    import torch
    M, N, K = 2048, 4096, 16384          # prefill needs 64 MB of bf16 X scratch
    note("linear_noalloc oversize")
    b, _ = capi.workspace_size(capi.OP_LINEAR, M, [N], K)
    assert b > 32 << 20
    x = torch.zeros((M, K), dtype=torch.float32, device=dev)
    w = torch.zeros(capi.q8_0_bytes(N * K), dtype=torch.uint8, device=dev)
    y = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    code, msg = capi.linear_noalloc_status(x, w, None, y, M, N, K)
    torch.cuda.synchronize()
    assert code == 4 and "no-allocation" in msg and str(b) in msg
    assert bool((y == 7.0).all())     # nothing was launched


def test_noalloc_back_to_back_split_k(dev):
    """Three MFMA decode calls with K splits, of different shapes (the hybrid decode's 8
    splits of 44 blocks, then split-K with 8 and 16 splits; different tile counts),
    enqueued on one stream with no synchronisation between them: each resets the
    counters it used before the next starts, and each matches mle_q8_0_linear."""
    import torch
    shapes = [(8, 4096, 11008, False), (4, 1024, 4096, True), (16, 2048, 8192, False)]
    stream = torch.cuda.Stream()
    ops, outs = [], []
    for i, (M, N, K, bias) in enumerate(shapes):
        ops.append(_operands(dev, 300 + 10 * i, M, N, K, bias))
        outs.append(empty_f32((M, N), dev))
    torch.cuda.synchronize()
    note("linear_noalloc: three calls with K splits back to back on one stream")
    with torch.cuda.stream(stream):
        for (M, N, K, _b), (dx, dw, db), y in zip(shapes, ops, outs):
            capi.linear_noalloc(dx, dw, db, y, M, N, K, stream=stream)
    stream.synchronize()
    for (M, N, K, _b), (dx, dw, db), y in zip(shapes, ops, outs):
        want = empty_f32((M, N), dev)
        capi.linear(dx, dw, db, want, M, N, K)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        assert torch.equal(y, want), (M, N, K)


def test_noalloc_under_graph_capture_fresh_process():
    """In a fresh process (the library's per-device scratch not yet set up): the first
    no-allocation call, made under graph capture, is refused; after one eager call a
    captured call with K splits (the hybrid decode) replays bit-identical to the eager
    result, with eager
    no-allocation calls of another shape on the same stream between the replays."""
    child = os.path.join(os.path.dirname(__file__), "noalloc_capture_child.py")
    note("linear_noalloc under graph capture (child process)")
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(
        [os.path.dirname(os.path.dirname(os.path.abspath(__file__))), env.get("PYTHONPATH", "")])
    p = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True,
                       timeout=240, env=env)
    print(p.stdout[-3000:], p.stderr[-3000:])
    assert p.returncode == 0, p.stderr[-2000:]
    assert "noalloc capture child: OK" in p.stdout
