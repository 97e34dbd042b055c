"""Shared test helpers: seeded inputs, paired host/device views, comparisons."""
from __future__ import annotations

import numpy as np

import oracle as orc

F32, F16, I32 = 0, 1, 26


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def uniform(seed: int, n: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    return rng(seed).uniform(lo, hi, n).astype(np.float32)


def normal(seed: int, n: int, sigma: float = 1.0) -> np.ndarray:
    return (rng(seed).standard_normal(n, dtype=np.float64) * sigma).astype(np.float32)


def row_major_nb(ne, elem=4):
    nb = [elem]
    for d in range(1, 4):
        nb.append(nb[-1] * ne[d - 1])
    return nb


def span_elems(ne, nb, elem=4):
    """Elements a (ne, nb) view spans (nb[0] == 0 -> row-major)."""
    if nb[0] == 0:
        nb = row_major_nb(ne, elem)
    return (sum((ne[d] - 1) * nb[d] for d in range(4)) + elem) // elem


class Pair:
    """One operand given to both the oracle (numpy buffer) and the product
    (a device copy of the same bytes)."""

    def __init__(self, buf: np.ndarray, ne, nb=None, dtype=None, data_bytes=None):
        self.host = np.ascontiguousarray(buf)
        self.ne = [int(x) for x in ne]
        elem = self.host.itemsize
        self.nb = row_major_nb(self.ne, elem) if nb is None else [int(x) for x in nb]
        if dtype is None:
            dtype = I32 if self.host.dtype == np.int32 else (F16 if elem == 2 else F32)
        self.dtype = dtype
        self.data_bytes = data_bytes
        self.dev = None

    def oview(self) -> orc.OView:
        return orc.view(self.host, self.ne, self.nb, self.dtype, self.data_bytes)

    def to(self, device):
        import torch

        self.dev = torch.from_numpy(self.host.copy()).to(device)
        return self

    def pview(self, mut=False):
        import emel_hip

        lay = emel_hip.Layout(self.dtype, self.ne, self.nb)
        cls = emel_hip.TensorViewMut if mut else emel_hip.TensorView
        return cls(self.dev, lay, self.data_bytes)

    def result(self) -> np.ndarray:
        return self.dev.cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32)


def assert_bits_equal(got: np.ndarray, want: np.ndarray, what: str = ""):
    """Bit-exact comparison; any NaN matches any NaN."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
    if not same.all():
        idx = np.flatnonzero(~same)
        i = idx[0]
        raise AssertionError(
            f"{what}: {idx.size} of {got.size} elements differ; first at {i}: "
            f"got {got.flat[i]!r} ({bits(got).flat[i]:08x}) want {want.flat[i]!r} ({bits(want).flat[i]:08x})"
        )


def assert_close_rel(got: np.ndarray, want: np.ndarray, rtol: float, what: str = "", atol: float = 0.0):
    """|got - want| <= rtol * |want| + atol elementwise; NaN matches NaN."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    nan = np.isnan(got) & np.isnan(want)
    with np.errstate(invalid="ignore"):
        ok = nan | (got == want) | (np.abs(got - want) <= rtol * np.abs(want) + atol)
    if not ok.all():
        i = np.flatnonzero(~ok)[0]
        raise AssertionError(f"{what}: {int((~ok).sum())} elements outside rtol={rtol}; first at {i}: "
                             f"got {got.flat[i]!r} want {want.flat[i]!r}")


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in units of f32 ulps on the ordered integer line."""
    def ordered(x):
        i = np.ascontiguousarray(x, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(ordered(a) - ordered(b))
