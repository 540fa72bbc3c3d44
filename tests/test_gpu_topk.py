"""GPU parity of mle_top_tokens_f32 against a numpy restatement of the reference's
Sampler::get_top_tokens (src/runtime/sampler.cpp:141-197): temperature scaling by
1/temperature, softmax exp(v - max) * (1 / sum), top-n by probability.

The restatement below sorts with numpy (value descending, index ascending) and
computes the softmax in float32; the ids must match exactly wherever probabilities
are distinct, the probabilities within 1e-5 relative (the device adds the row's
exponentials in another order than the reference's sequential float sum).  Ties,
which std::partial_sort leaves unordered, go to the lower index on the device.
"""
import numpy as np
import pytest

from helpers import note, to_dev
from llmengine_amd import capi
from llmengine_amd import synthetic as S

pytestmark = pytest.mark.gpu


def ref_top_tokens(row, top_n, temperature):
    """get_top_tokens for one row: (ids, probs), or the uniform case."""
    n = row.size
    k = min(top_n, n)
    v = row.astype(np.float32)
    if temperature > 0 and temperature != 1:
        v = (v * (np.float32(1) / np.float32(temperature))).astype(np.float32)
    mx = np.float32(np.max(v)) if not np.isnan(v).any() else np.float32(np.nan)
    uniform = (np.arange(k, dtype=np.int32), np.full(k, np.float32(1) / np.float32(n)))
    if not np.isfinite(mx):
        return uniform
    e = np.exp((v - mx).astype(np.float32)).astype(np.float32)
    s = np.float32(e.sum(dtype=np.float32))
    if not np.isfinite(s) or s <= 0:
        return uniform
    p = (e * (np.float32(1) / s)).astype(np.float32)
    order = np.lexsort((np.arange(n), -v.astype(np.float64)))[:k]
    return order.astype(np.int32), p[order]


def run(x, rows, n, top_n, temperature, dev):
    import torch
    k = min(top_n, n)
    ids = torch.full((rows, k), -1, dtype=torch.int32, device=dev)
    probs = torch.full((rows, k), float("nan"), dtype=torch.float32, device=dev)
    capi.top_tokens(to_dev(x, dev), rows, n, top_n, ids, probs, temperature)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), probs.cpu().numpy()


@pytest.mark.parametrize("rows,n,top_n,temperature", [
    (1, 1, 1, 1.0), (1, 7, 5, 1.0), (1, 5, 10, 1.0), (3, 2048, 40, 0.7), (2, 2049, 128, 1.0),
    (1, 151936, 40, 0.8), (4, 151936, 128, 1.0), (2, 100000, 1, 0.0), (2, 32000, 50, 1.5)])
def test_top_tokens_match_reference(dev, rows, n, top_n, temperature):
    note(f"top_tokens rows={rows} n={n} top_n={top_n} t={temperature}")
    x = (S.activations(400 + n + top_n, (rows, n)) * np.float32(3)).astype(np.float32)
    ids, probs = run(x, rows, n, top_n, temperature, dev)
    for r in range(rows):
        want_ids, want_p = ref_top_tokens(x[r], top_n, temperature)
        assert np.array_equal(ids[r], want_ids), r
        np.testing.assert_allclose(probs[r], want_p, rtol=1e-5, atol=0)


def test_top_tokens_first_is_argmax(dev):
    import torch
    rows, n = 3, 151936
    x = S.activations(410, (rows, n))
    ids, _ = run(x, rows, n, 8, 1.0, dev)
    idx = torch.empty(rows, dtype=torch.int32, device=dev)
    capi.argmax(to_dev(x, dev), rows, n, idx)
    torch.cuda.synchronize()
    assert np.array_equal(ids[:, 0], idx.cpu().numpy())


def test_top_tokens_ties_and_special_rows(dev):
    n = 10_000
    x = np.full((6, n), -1.0, dtype=np.float32)
    x[0, [4000, 17, 9000]] = 3.0                     # tie: 17, 4000, 9000 in that order
    x[1, :] = -np.inf
    x[1, 1234] = 2.0                                 # the only finite logit: probability 1
    x[2, 7] = np.nan                                 # NaN: uniform
    x[3, 99] = np.inf                                # +Inf maximum: uniform
    x[4, :] = -np.inf                                # all -Inf: uniform
    x[5, 1::2] = 0.5                                 # 5000-way tie at the top
    note("top_tokens ties and special rows")
    ids, probs = run(x, 6, n, 6, 1.0, dev)
    assert ids[0, :3].tolist() == [17, 4000, 9000]
    np.testing.assert_allclose(probs[0, :3], ref_top_tokens(x[0], 6, 1.0)[1][:3], rtol=1e-5)
    assert ids[1, 0] == 1234 and probs[1, 0] == 1.0 and np.all(probs[1, 1:] == 0.0)
    for r in (2, 3, 4):
        assert ids[r].tolist() == list(range(6)), r
        assert np.all(probs[r] == np.float32(1) / np.float32(n)), r
    assert ids[5].tolist() == [1, 3, 5, 7, 9, 11]
    np.testing.assert_allclose(probs[5], ref_top_tokens(x[5], 6, 1.0)[1], rtol=1e-5)


def test_top_tokens_lm_head_pipeline(dev, orc):
    """lm_head [151936, 896] Linear at M=2 then top-40: the device's candidates equal
    the reference restatement applied to the oracle's logits wherever neighbouring
    logits are farther apart than the Linear's error."""
    import torch
    V, H = 151936, 896
    w = S.q8_0_weight(420, V, H)[0]
    x = S.activations(421, (2, H))
    logits = torch.empty((2, V), dtype=torch.float32, device=dev)
    capi.linear(to_dev(x, dev), to_dev(w, dev), None, logits, 2, V, H)
    ids, probs = run(logits.cpu().numpy(), 2, V, 40, 0.8, dev)
    want = orc.linear(x, w, None, 2, V, H)
    for r in range(2):
        wi, wp = ref_top_tokens(want[r], 40, 0.8)
        v = np.sort(want[r])[::-1][:41]
        clear = np.all(np.diff(v) < -1e-4 * np.abs(v[:-1]))
        if clear:
            assert np.array_equal(ids[r], wi), r
            np.testing.assert_allclose(probs[r], wp, rtol=2e-4)
