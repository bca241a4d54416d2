"""GPU check of gdn_qlinear_noalloc, the no-allocation variant of gdn_qlinear: through the C
ABI, its outputs must equal gdn_qlinear's (same kernels, same arithmetic: bit for bit) on two
calls in a row, the second with a smaller operand, so stale scratch contents from the first
call cannot leak into the second (the prep kernel rewrites every scratch row it uses,
padding rows included)."""
from __future__ import annotations

import numpy as np
import pytest

from _util import log_case, to_dev, to_np

pytestmark = pytest.mark.gpu


def _mats(O, gdn, dev, L, ns, K, seed):
    rng = np.random.default_rng(seed)
    mats = []
    for n in ns:
        w = rng.integers(0, 2 ** 32, (L, n, K // 8), dtype=np.uint64).astype(np.uint32)
        s = O.to_bf16(rng.uniform(0.002, 0.03, (L, n, K // 64)).astype(np.float32))
        b = O.to_bf16(rng.uniform(-0.2, 0.2, (L, n, K // 64)).astype(np.float32))
        if L == 1:
            w, s, b = w[0], s[0], b[0]
        mats.append(gdn.QuantLinear(to_dev(w.view(np.int32), dev), to_dev(s, dev), to_dev(b, dev)))
    return mats


def _same(ys_a, ys_b, what):
    for i, (a, b) in enumerate(zip(ys_a, ys_b)):
        ga, gb = to_np(a), to_np(b)
        nd = int(np.count_nonzero(ga != gb))
        print(f"  {what} segment {i}: {ga.size} outputs, {nd} differ", flush=True)
        assert nd == 0, (what, i)


def test_qlinear_noalloc_equals_qlinear_two_calls(O, gdn, dev):
    import torch
    # call 1: a verify block through in_proj (four segments), M = 40, K = 5120
    log_case("qlinear_noalloc call 1: in_proj 4 segments, M=40, K=5120")
    K = 5120
    mats = _mats(O, gdn, dev, 1, [2048, 1024, 48, 48], K, seed=501)
    x = to_dev(O.to_bf16(np.random.default_rng(502).standard_normal((40, K)).astype(np.float32)), dev)
    ref = gdn.qlinear(mats, x)
    got = gdn.qlinear_noalloc(mats, x)
    torch.cuda.synchronize()
    _same(got, ref, "call 1")
    # call 1b: 8 layers of the in_proj row count at M = 40 (K = 1024): enough 256-row
    # workgroups for the kernel whose waves share the operand through LDS
    log_case("qlinear_noalloc call 1b: in_proj rows x 8 layers, M=40, K=1024 (operand-sharing kernel)")
    mats1b = _mats(O, gdn, dev, 8, [10240, 6144, 48, 48], 1024, seed=508)
    x1b = to_dev(O.to_bf16(np.random.default_rng(509).standard_normal((8, 40, 1024)).astype(np.float32)), dev)
    ref1b = gdn.qlinear(mats1b, x1b, n_layers=8)
    got1b = gdn.qlinear_noalloc(mats1b, x1b, n_layers=8)
    torch.cuda.synchronize()
    _same(got1b, ref1b, "call 1b")
    # call 2: smaller -- M = 5 (one 16-row tile, rows 5..15 are zero padding in the scratch
    # that call 1 filled with data), K = 1024, with the GatedRMSNorm prologue
    log_case("qlinear_noalloc call 2: norm + out_proj, M=5, K=1024, N=300")
    K2, M2 = 1024, 5
    rng = np.random.default_rng(503)
    o = to_dev((rng.standard_normal((M2, K2)) * 0.3).astype(np.float32), dev)
    z = to_dev(O.to_bf16(rng.standard_normal((M2, K2)).astype(np.float32)), dev)
    gamma = to_dev(rng.uniform(0.5, 1.5, 128).astype(np.float32), dev)
    mats2 = _mats(O, gdn, dev, 1, [300], K2, seed=504)
    ref2 = gdn.qlinear(mats2, norm=(o, z, gamma, 1e-6))
    got2 = gdn.qlinear_noalloc(mats2, norm=(o, z, gamma, 1e-6))
    torch.cuda.synchronize()
    _same(got2, ref2, "call 2")
    # and the largest one-layer operand the scratch holds, M = 512, K = 8192 (the whole
    # scratch), then the GEMV path (no scratch at all)
    log_case("qlinear_noalloc call 3: M=512, K=8192, N=64 (the whole scratch)")
    mats3 = _mats(O, gdn, dev, 1, [64], 8192, seed=505)
    x3 = to_dev(O.to_bf16(np.random.default_rng(506).standard_normal((512, 8192)).astype(np.float32)), dev)
    ref3 = gdn.qlinear(mats3, x3)
    got3 = gdn.qlinear_noalloc(mats3, x3)
    torch.cuda.synchronize()
    _same(got3, ref3, "call 3")
    log_case("qlinear_noalloc call 4: GEMV path, M=2, K=5120")
    x4 = to_dev(O.to_bf16(np.random.default_rng(507).standard_normal((2, K)).astype(np.float32)), dev)
    ref4 = gdn.qlinear(mats, x4)
    got4 = gdn.qlinear_noalloc(mats, x4)
    torch.cuda.synchronize()
    _same(got4, ref4, "call 4")


def test_qlinear_noalloc_rejects_oversize_on_gpu(O, gdn, dev):
    import torch
    log_case("qlinear_noalloc: 2 layers x M=512 x K=8192 exceeds the scratch")
    x = torch.zeros((2, 512, 8192), dtype=torch.bfloat16, device=dev)
    mats = _mats(O, gdn, dev, 2, [16], 8192, seed=508)
    with pytest.raises(gdn.GdnError, match="scratch"):
        gdn.qlinear_noalloc(mats, x, n_layers=2)
