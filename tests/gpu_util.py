"""Helpers shared by the GPU parity tests (imported by tests only)."""
import numpy as np
import torch


def dev():
    return torch.device("cuda", 0)


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def to_host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def random_int4(rng, rows, width):
    return rng.integers(-7, 8, size=(rows, width), dtype=np.int8)


def assert_bits_equal(actual, expected, what=""):
    a = np.ascontiguousarray(actual)
    e = np.ascontiguousarray(expected)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    if a.dtype.kind == "f":
        bad = np.flatnonzero(a.view(np.uint32 if a.itemsize == 4 else np.uint16).ravel()
                             != e.view(np.uint32 if e.itemsize == 4 else np.uint16).ravel())
    else:
        bad = np.flatnonzero(a.ravel() != e.ravel())
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {a.size} differ; first at {i}: "
                             f"{a.ravel()[i]!r} vs {e.ravel()[i]!r}")
