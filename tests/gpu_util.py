"""Helpers shared by the GPU parity tests (imported only when a GPU test runs)."""
import numpy as np

F32 = np.float32
EPS = float(np.finfo(np.float32).eps)


def dev():
    import torch

    return torch.device("cuda:0")


def to_dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def host(t):
    return t.detach().cpu().numpy()


def assert_bitwise(got, want, label=""):
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, f"{label}: shape {got.shape} vs {want.shape}"
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    # NaNs compare by class, everything else by bits (signed zeros included).
    same = (gb == wb) | (np.isnan(got) & np.isnan(want))
    if not same.all():
        i = int(np.flatnonzero(~same.ravel())[0])
        raise AssertionError(f"{label}: {int((~same).sum())} of {same.size} differ; first at {np.unravel_index(i, got.shape)}: "
                             f"{got.ravel()[i]!r} vs {want.ravel()[i]!r}")


def max_rel(got, want):
    """max |got - want| / max |want| over the tensor (the FP32 tolerance metric)."""
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


def oracle_threads():
    """Threads for the CPU oracle: the CPUs this process may run on, at most 16
    (the host share of a one-GPU job)."""
    import os

    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))
