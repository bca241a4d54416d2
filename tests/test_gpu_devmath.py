"""The front ends' device math on every bf16 input, bit for bit against the oracle.

The front ends' SiLU takes its sigmoid from the hardware 2^x and reciprocal for |y| < 8
(the exact path otherwise), and the l2norm's reciprocal square root from v_rsq_f32 unless
the result lies within 4 ulp of a bf16 rounding midpoint. Both inputs are bf16 values, so
the domain is finite and these tests are exhaustive: SiLU over all 65,536 bf16 patterns
(every value in a batch of eight copies of itself, so each takes its own path), and the
reciprocal square root over every positive finite bf16 value, subnormals included. The
oracle's silu is rb(y * rb(sigmoid(y))) and its reciprocal square root rb(1 / sqrtf(d))
(ops.cpp:20, 27-30). The probe library is tests/cpp/libdevmath_probe.so.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from _util import log_case

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "libdevmath_probe.so")


@pytest.fixture(scope="module")
def probe():
    if not os.path.exists(PROBE):
        pytest.fail(f"{PROBE} is missing: build it with __graft_entry__.build()")
    L = ctypes.CDLL(PROBE)
    for name in ("probe_silu_bf_batch", "probe_rsqrt_bf"):
        getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        getattr(L, name).restype = ctypes.c_int
    return L


def _bf16_values(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _round(O, x: np.ndarray) -> np.ndarray:
    """Oracle bf16 rounding (RNE), kept in fp32."""
    return _bf16_values(O.to_bf16(x.astype(np.float32)).view(np.uint16))


def _same_bits(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Equal fp32 bit patterns, or both NaN."""
    return (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))


def test_silu_batch_every_bf16(O, probe, dev):
    import torch
    log_case("device silu_bf_batch on all 65536 bf16 patterns")
    y = _bf16_values(np.arange(1 << 16, dtype=np.uint32).astype(np.uint16))
    sig = np.array([O.lib().gdno_sigmoidf(float(v)) for v in y], dtype=np.float32)
    want = _round(O, y * _round(O, sig))
    yd = torch.from_numpy(np.repeat(y, 8)).to(dev)
    out = torch.empty_like(yd)
    assert probe.probe_silu_bf_batch(yd.data_ptr(), out.data_ptr(), y.size) == 0
    got = out.cpu().numpy().reshape(-1, 8)
    assert all(_same_bits(got[:, j], got[:, 0]).all() for j in range(1, 8))
    ok = _same_bits(got[:, 0], want)
    fast = np.abs(y) < 8
    print(f"  {y.size} patterns ({int(fast.sum())} on the fast path), mismatches {int((~ok).sum())}", flush=True)
    assert ok.all(), y[~ok][:8]


def test_rsqrt_every_positive_bf16(O, probe, dev):
    import torch
    log_case("device rsqrt_bf on every positive finite bf16")
    bits = np.arange(1, 0x7F80, dtype=np.uint32).astype(np.uint16)   # +subnormals .. max finite
    d = _bf16_values(bits)
    want = _round(O, np.array([O.lib().gdno_rsqrtf(float(v)) for v in d], dtype=np.float32))
    dd = torch.from_numpy(d).to(dev)
    out = torch.empty_like(dd)
    assert probe.probe_rsqrt_bf(dd.data_ptr(), out.data_ptr(), d.size) == 0
    got = out.cpu().numpy()
    ok = _same_bits(got, want)
    print(f"  {d.size} values, mismatches {int((~ok).sum())}", flush=True)
    assert ok.all(), d[~ok][:8]
