"""Helpers shared by the GPU tests: host<->device copies and error metrics."""
from __future__ import annotations

import hashlib
import sys

import numpy as np


def note(msg: str) -> None:
    """Print the case about to run (flushed) so a failing GPU step names itself."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def empty_f32(shape, dev):
    import torch
    # filled with NaN so that an output the kernel forgets to write fails the check
    return torch.full(shape, float("nan"), dtype=torch.float32, device=dev)


def to_host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def rel_l2(a, ref) -> float:
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(a - ref) / (den if den > 0 else 1.0))


def assert_bitexact(got, want, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    diff = np.nonzero(bits(got)[~wn] != bits(want)[~wn])[0]
    assert diff.size == 0, f"{what}: {diff.size} values differ, first at {diff[:5]}"
