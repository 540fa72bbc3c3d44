"""Linear launches captured in a HIP graph (torch.cuda.CUDAGraph) on a stream whose
workspace was reserved beforehand (mle_q8_0_workspace_size + mle_workspace_reserve):
capture allocates and synchronises nothing, and every replay -- on the capturing stream
with eager launches of other shapes after it, on the default stream while eager launches
of another shape run on the capturing stream at the same time (captured calls use the
stream's graph workspace, which no eager call shares), and after a later eager call has
outgrown the reservation -- gives the eager results bit for bit.  Shapes:
the split-K MFMA decode (M = 16, 22 splits), the tiled FP32 GEMV (M = 1), the bf16 GEMM
with its X pre-pass (M = 96), the row-range MFMA decode (M = 4 on 512 tiled row
groups, no workspace) and the hybrid MFMA decode (M = 8 on tiled rows of 11008
elements, 8 splits through the workspace).  The kernels
reset their split-K counters themselves and the workspace counters were cleared by a
fill kernel at allocation, so no memset node enters the graph.
"""
import numpy as np
import pytest

from helpers import empty_f32, hybrid_decode, note, rel_l2, rows_decode, to_dev, to_host
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu


def test_linear_graph_replays_match_eager(dev, orc):
    import torch
    shapes = [(16, 1024, 11008, False), (1, 512, 4096, True), (96, 384, 1024, False),
              (4, 8192, 4096, True), (8, 1024, 11008, True)]
    assert rows_decode(4, 8192, 4096)  # the fourth shape takes the row-range kernel
    assert hybrid_decode(8, 1024, 11008)  # the last one the hybrid kernel
    stream = torch.cuda.Stream()
    need_b = need_c = 0
    cases = []
    for i, (M, N, K, tiled) in enumerate(shapes):
        w = S.q8_0_weight(150 + i, N, K)[0]
        x = S.activations(151 + i, (M, K))
        dw = to_dev(w, dev)
        if tiled:
            t = torch.empty(capi.tiled_bytes(N, K), dtype=torch.uint8, device=dev)
            capi.tile(dw, t, N, K)
            dw = t
        b, c = capi.workspace_size(capi.OP_LINEAR, M, [N], K, tiled)
        need_b, need_c = max(need_b, b), max(need_c, c)
        cases.append((M, N, K, tiled, dw, to_dev(x, dev), orc.sgemm_nt(x, w, M, N, K)))
    # The eager launch made between replays fits the reservation too, so the
    # generation checks below see no growth.
    b, c = capi.workspace_size(capi.OP_LINEAR, 4, [2048], 4096)
    need_b, need_c = max(need_b, b), max(need_c, c)
    capi.workspace_reserve(need_b, need_c, stream=stream)
    torch.cuda.synchronize()
    gen0 = capi.workspace_info(stream)[2]

    def run_all(outs):
        for (M, N, K, tiled, dw, dx, _), y in zip(cases, outs):
            (capi.linear_tiled if tiled else capi.linear)(dx, dw, None, y, M, N, K,
                                                          stream=stream)

    eager = [empty_f32((M, N), dev) for (M, N, *_r) in cases]
    with torch.cuda.stream(stream):
        run_all(eager)
    stream.synchronize()
    for (M, N, K, tiled, _dw, _dx, want), y in zip(cases, eager):
        assert rel_l2(to_host(y), want) <= (1e-2 if M >= 64 else 1e-5), (M, N, K)

    note("capture Linear launches in a HIP graph")
    graph_out = [empty_f32((M, N), dev) for (M, N, *_r) in cases]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run_all(graph_out)
    assert capi.workspace_info(stream)[2] == gen0  # nothing (re)allocated

    other = empty_f32((4, 2048), dev)
    wo = to_dev(S.q8_0_weight(160, 2048, 4096)[0], dev)
    xo = to_dev(S.activations(161, (4, 4096)), dev)
    for rep in range(4):
        for y in graph_out:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):  # replay() launches on the current stream
            g.replay()
        # eager work of another shape on the same stream between replays (ordered
        # after the replay: both use this stream's workspace)
        capi.linear(xo, wo, None, other, 4, 2048, 4096, stream=stream)
        torch.cuda.synchronize()
        assert capi.workspace_info(stream)[2] == gen0
        for (M, N, *_r), a, b in zip(cases, eager, graph_out):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), (rep, M, N)
    assert capi.workspace_info(stream)[2] == gen0

    # Replays on the default stream, not ordered with eager split-K calls enqueued on the
    # capturing stream right after them: the two may run at the same time, each on its
    # own workspace.
    note("replay on the default stream beside eager calls on the capturing stream")
    xe = to_dev(S.activations(164, (8, 11008)), dev)
    we = to_dev(S.q8_0_weight(165, 1024, 11008)[0], dev)
    ye = [empty_f32((8, 1024), dev) for _ in range(3)]
    want_e = empty_f32((8, 1024), dev)
    capi.linear(xe, we, None, want_e, 8, 1024, 11008, stream=stream)
    torch.cuda.synchronize()
    for rep in range(4):
        for y in graph_out:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()  # current stream: the default stream
        for y in ye:
            capi.linear(xe, we, None, y, 8, 1024, 11008, stream=stream)
        torch.cuda.synchronize()
        for (M, N, *_r), a, b in zip(cases, eager, graph_out):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), ("default", rep, M, N)
        for y in ye:
            assert torch.equal(y.view(torch.int32), want_e.view(torch.int32)), ("eager", rep)

    # A call that outgrows the reservation replaces the workspace buffers but keeps
    # the old ones, which the graph's kernels still point to: replays stay exact.
    note("grow the workspace after capture, then replay")
    Mb, Nb, Kb = 512, 256, 11008
    xb = S.activations(162, (Mb, Kb))
    wb = S.q8_0_weight(163, Nb, Kb)[0]
    yb = empty_f32((Mb, Nb), dev)
    capi.linear(to_dev(xb, dev), to_dev(wb, dev), None, yb, Mb, Nb, Kb, stream=stream)
    torch.cuda.synchronize()
    assert capi.workspace_info(stream)[2] > gen0
    rows = np.arange(0, Nb, 17)
    w_rows = np.ascontiguousarray(wb.reshape(Nb, -1)[rows]).reshape(-1)  # rows are contiguous
    want_b = orc.sgemm_nt(xb, w_rows, Mb, rows.size, Kb)
    assert rel_l2(to_host(yb)[:, rows], want_b) <= 1e-2
    for y in graph_out:
        y.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.replay()
    torch.cuda.synchronize()
    for (M, N, *_r), a, b in zip(cases, eager, graph_out):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), ("after growth", M, N)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_capture_without_reservation_is_refused(dev):
    """A Linear that would have to allocate its workspace while its stream is capturing
    returns RuntimeError with a message naming the reservation, instead of calling
    hipMalloc inside the capture."""
    import torch
    M, N, K = 8, 512, 11008
    dw = to_dev(S.q8_0_weight(170, N, K)[0], dev)
    dx = to_dev(S.activations(171, (M, K)), dev)
    y = empty_f32((M, N), dev)
    stream = torch.cuda.Stream()  # fresh: no workspace yet
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(capi.Q8_0Error) as err:
        with torch.cuda.graph(g, stream=stream):
            capi.linear(dx, dw, None, y, M, N, K, stream=stream)
    assert err.value.code == 6 and "reserve it before capture" in str(err.value)
    assert capi.workspace_info(stream)[2] == 0
