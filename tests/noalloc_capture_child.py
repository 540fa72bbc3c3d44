"""Child process of test_zz_no_alloc.py (not collected by pytest): exercises
mle_q8_0_linear_noalloc under HIP graph capture in a process where the library's
static device scratch has not been used yet.  Prints "noalloc capture child: OK"."""
import warnings

import torch

from llmengine_amd import capi
from llmengine_amd import synthetic as S


def dev_tensor(a):
    return torch.from_numpy(a).to("cuda:0")


def main():
    dev = "cuda:0"
    M, N, K = 8, 4096, 11008            # hybrid decode (8 K splits through the scratch)
    Mo, No, Ko = 4, 1024, 4096          # a split-K shape for the eager calls
    x = dev_tensor(S.activations(401, (M, K)))
    w = dev_tensor(S.q8_0_weight(402, N, K)[0])
    xo = dev_tensor(S.activations(403, (Mo, Ko)))
    wo = dev_tensor(S.q8_0_weight(404, No, Ko)[0])
    y = torch.full((M, N), float("nan"), device=dev)
    yo = torch.full((Mo, No), float("nan"), device=dev)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()

    print("[child] first call under capture", flush=True)
    g0 = torch.cuda.CUDAGraph()
    refused = None
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        try:
            with torch.cuda.graph(g0, stream=stream):
                capi.linear_noalloc(x, w, None, y, M, N, K, stream=stream)
        except capi.Q8_0Error as e:
            refused = e
    assert refused is not None and refused.code == 6, refused
    assert "must not be captured" in str(refused), str(refused)

    print("[child] eager reference and first eager no-allocation call", flush=True)
    want = torch.full((M, N), float("nan"), device=dev)
    capi.linear(x, w, None, want, M, N, K)
    want_o = torch.full((Mo, No), float("nan"), device=dev)
    capi.linear(xo, wo, None, want_o, Mo, No, Ko)
    with torch.cuda.stream(stream):
        capi.linear_noalloc(x, w, None, y, M, N, K, stream=stream)
    torch.cuda.synchronize()
    assert torch.equal(y, want)

    print("[child] capture a no-allocation call with K splits", flush=True)
    yg = torch.full((M, N), float("nan"), device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        capi.linear_noalloc(x, w, None, yg, M, N, K, stream=stream)
    for rep in range(4):
        yg.fill_(float("nan"))
        yo.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g.replay()
            capi.linear_noalloc(xo, wo, None, yo, Mo, No, Ko, stream=stream)
        torch.cuda.synchronize()
        assert torch.equal(yg, want), rep
        assert torch.equal(yo, want_o), rep
    print("noalloc capture child: OK", flush=True)


if __name__ == "__main__":
    main()
