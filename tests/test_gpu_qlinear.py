"""GPU parity of gdn_qlinear -- Linear::operator() for 4-bit weights
(cpp/src/model.cpp:356-372) and the GatedRMSNorm + out_proj pair (model.cpp:350-354,
626-641) -- against the oracle's fp64 dequantize-and-dot.

Tolerance: the result is rounded to bf16 once (half an ulp: at most 2^-8 relative), and the fp32
accumulation (products of x with the offset bf16 values 128 + nibble, per 32-value piece)
adds at most 2^-20 of sum_k |x_k| (143 |s_k| + |b_k|), the magnitudes it accumulates. The
test allows 2^-8 |y| plus that bound. MLX's own accumulation order is unpinned at bit
level; the reference rounds its fp32 result to bf16 as this does.
"""
from __future__ import annotations

import numpy as np
import pytest

from _util import bf16_to_f32, log_case, to_dev, to_np

pytestmark = pytest.mark.gpu


def quant_inputs(O, L, M, N, K, seed):
    rng = np.random.default_rng(seed)
    x = O.to_bf16(rng.standard_normal((L, M, K)).astype(np.float32))
    w = rng.integers(0, 2 ** 32, (L, N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = O.to_bf16(rng.uniform(0.002, 0.03, (L, N, K // 64)).astype(np.float32))
    b = O.to_bf16(rng.uniform(-0.2, 0.2, (L, N, K // 64)).astype(np.float32))
    return x, w, s, b


def dev_mat(gdn, dev, w, s, b):
    return gdn.QuantLinear(to_dev(w.view(np.int32), dev), to_dev(s, dev), to_dev(b, dev))


def bound(O, x_bf16, s, b):
    """Per-output fp32 accumulation bound: 2^-20 sum_k |x_k| (143 |s_k| + |b_k|)."""
    xa = np.abs(bf16_to_f32(x_bf16)).astype(np.float64)                 # (M, K)
    mag = 143.0 * np.abs(bf16_to_f32(s)) + np.abs(bf16_to_f32(b))        # (N, K/64)
    return 2.0 ** -20 * (xa @ np.repeat(mag, 64, axis=1).T)              # (M, N)


def check(got_bf16, ref, tol_abs, what):
    got = bf16_to_f32(got_bf16).astype(np.float64)
    err = np.abs(got - ref)
    lim = 2.0 ** -8 * np.abs(ref) + tol_abs
    worst = (err / np.maximum(lim, 1e-30)).max()
    print(f"  {what}: max |err| {err.max():.3e}, worst err / limit {worst:.3f}", flush=True)
    assert np.all(np.isfinite(got)), what
    assert np.all(err <= lim), what


@pytest.mark.parametrize("M,N,K", [(1, 200, 1024), (2, 96, 5120), (4, 130, 6144), (3, 64, 8192),
                                   (1, 48, 2048), (4, 17, 4096)])
def test_qlinear_single_matrix(O, gdn, dev, M, N, K):
    import torch
    log_case(f"qlinear M={M} N={N} K={K}")
    x, w, s, b = quant_inputs(O, 1, M, N, K, seed=N + K + M)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])], to_dev(x[0], dev))
    torch.cuda.synchronize()
    ref = O.qlinear(x[0], w[0], s[0], b[0])
    check(to_np(y), ref, bound(O, x[0], s[0], b[0]), "y")


def test_qlinear_in_proj_four_matrices_two_layers(O, gdn, dev):
    """The DeltaNet layer's in_proj_qkv (10240), in_proj_z (6144), in_proj_a, in_proj_b (48)
    on one x of 5120 (model.cpp:587, 608-609, 626), two layers stacked, B=1."""
    import torch
    log_case("qlinear in_proj 4 segments x 2 layers, K=5120")
    L, M, K = 2, 1, 5120
    ns = [10240, 6144, 48, 48]
    mats, host = [], []
    x = None
    for i, n in enumerate(ns):
        xi, w, s, b = quant_inputs(O, L, M, n, K, seed=100 + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w, s, b))
        host.append((w, s, b))
    ys = gdn.qlinear(mats, to_dev(x, dev), n_layers=L)
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        got = to_np(y)
        for l in range(L):
            ref = O.qlinear(x[l], w[l], s[l], b[l])
            check(got[l], ref, bound(O, x[l], s[l], b[l]), f"segment {i} layer {l}")


def test_qlinear_gated_rmsnorm_prologue(O, gdn, dev):
    """out_proj(GatedRMSNorm(o, z)) in one call (model.cpp:626-641): o fp32 (M, 6144), z bf16,
    gamma (128); against the oracle's norm (bf16 operand) then its fp64 product. A one-ulp
    flip of an operand element between the two norms (fp32 reductions in different
    orders) moves y by at most 2^-8 |x_k w_k|; three such flips are allowed per output."""
    import torch
    log_case("qlinear out_proj with GatedRMSNorm, M=2, K=6144, N=5120")
    M, K, N = 2, 6144, 5120
    rng = np.random.default_rng(77)
    o = (rng.standard_normal((M, K)) * 0.3).astype(np.float32)
    z = O.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    gamma = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    _, w, s, b = quant_inputs(O, 1, M, N, K, seed=78)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])],
                       norm=(to_dev(o, dev), to_dev(z, dev), to_dev(gamma, dev), 1e-6))
    torch.cuda.synchronize()
    xn = O.gated_rmsnorm(o.reshape(M * 48, 128), z.reshape(M * 48, 128), gamma, 1e-6).reshape(M, K)
    ref = O.qlinear(xn, w[0], s[0], b[0])
    W = (np.abs(np.repeat(bf16_to_f32(s[0]), 64, axis=1)) * 15 + np.abs(np.repeat(bf16_to_f32(b[0]), 64, axis=1)))
    flip = 3 * 2.0 ** -8 * (np.abs(bf16_to_f32(xn)).max(axis=1, keepdims=True) * W.max(axis=1)[None, :])
    check(to_np(y), ref, bound(O, xn, s[0], b[0]) + flip, "y")


def test_qlinear_rejects_bad_arguments_on_gpu(gdn, dev):
    import torch
    x = torch.zeros((1, 5000), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((8, 625), dtype=torch.int32, device=dev)
    sb = torch.zeros((8, 78), dtype=torch.bfloat16, device=dev)
    with pytest.raises(gdn.GdnError, match="unsupported"):
        gdn.qlinear([gdn.QuantLinear(w, sb, sb)], x)


# ---- more than 4 rows: the MFMA path (operand in fragment order in a workspace) ----

@pytest.mark.parametrize("M,N,K", [(5, 200, 1024), (16, 96, 5120), (17, 130, 6144), (40, 64, 8192),
                                   (64, 48, 2048), (100, 17, 4096), (4, 72, 8192), (257, 40, 1024)])
def test_qlinear_mfma_single_matrix(O, gdn, dev, M, N, K):
    import torch
    log_case(f"qlinear (MFMA path) M={M} N={N} K={K}")
    x, w, s, b = quant_inputs(O, 1, M, N, K, seed=7 * N + K + M)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])], to_dev(x[0], dev))
    torch.cuda.synchronize()
    check(to_np(y), O.qlinear(x[0], w[0], s[0], b[0]), bound(O, x[0], s[0], b[0]), "y")


def test_qlinear_mfma_in_proj_verify_block(O, gdn, dev):
    """The layer's four in_proj matrices on a verify block's 40 rows (B=8, T=5), K=5120."""
    import torch
    log_case("qlinear (MFMA path) in_proj 4 segments, M=40, K=5120")
    M, K = 40, 5120
    ns = [10240, 6144, 48, 48]
    mats, host, x = [], [], None
    for i, n in enumerate(ns):
        xi, w, s, b = quant_inputs(O, 1, M, n, K, seed=200 + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w[0], s[0], b[0]))
        host.append((w[0], s[0], b[0]))
    ys = gdn.qlinear(mats, to_dev(x[0], dev))
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        check(to_np(y), O.qlinear(x[0], w, s, b), bound(O, x[0], s, b), f"segment {i}")


def test_qlinear_mfma_two_layers_two_segments(O, gdn, dev):
    import torch
    log_case("qlinear (MFMA path) 2 layers x 2 segments, M=24, K=2048")
    L, M, K = 2, 24, 2048
    mats, host, x = [], [], None
    for i, n in enumerate([100, 36]):
        xi, w, s, b = quant_inputs(O, L, M, n, K, seed=300 + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w, s, b))
        host.append((w, s, b))
    ys = gdn.qlinear(mats, to_dev(x, dev), n_layers=L)
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        got = to_np(y)
        for l in range(L):
            check(got[l], O.qlinear(x[l], w[l], s[l], b[l]), bound(O, x[l], s[l], b[l]), f"segment {i} layer {l}")


@pytest.mark.parametrize("M", [5, 17, 40, 64])
def test_qlinear_mfma_gated_rmsnorm_prologue(O, gdn, dev, M):
    """out_proj(GatedRMSNorm(o, z)) for M rows on the MFMA path (the norm applied while the
    operand goes to the workspace), same tolerance as the GEMV path's test."""
    import torch
    log_case(f"qlinear (MFMA path) out_proj with GatedRMSNorm, M={M}, K=6144, N=5120")
    K, N = 6144, 5120
    rng = np.random.default_rng(900 + M)
    o = (rng.standard_normal((M, K)) * 0.3).astype(np.float32)
    z = O.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    gamma = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    _, w, s, b = quant_inputs(O, 1, M, N, K, seed=901 + M)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])],
                       norm=(to_dev(o, dev), to_dev(z, dev), to_dev(gamma, dev), 1e-6))
    torch.cuda.synchronize()
    xn = O.gated_rmsnorm(o.reshape(M * 48, 128), z.reshape(M * 48, 128), gamma, 1e-6).reshape(M, K)
    ref = O.qlinear_blocked(xn, w[0], s[0], b[0])
    W = (np.abs(np.repeat(bf16_to_f32(s[0]), 64, axis=1)) * 15 + np.abs(np.repeat(bf16_to_f32(b[0]), 64, axis=1)))
    flip = 3 * 2.0 ** -8 * (np.abs(bf16_to_f32(xn)).max(axis=1, keepdims=True) * W.max(axis=1)[None, :])
    check(to_np(y), ref, bound(O, xn, s[0], b[0]) + flip, "y")


def test_qlinear_mfma_reuses_a_caller_workspace(O, gdn, dev):
    """One workspace, two calls in a row with different M; the second's result must not
    depend on what the first left there."""
    import torch
    log_case("qlinear (MFMA path) caller workspace reused, M=40 then M=9")
    K, N = 5120, 80
    ws = torch.empty(gdn.qlinear_workspace_size(40, K), dtype=torch.uint8, device=dev)
    for M, seed in ((40, 11), (9, 12)):
        x, w, s, b = quant_inputs(O, 1, M, N, K, seed=seed)
        (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])], to_dev(x[0], dev), workspace=ws)
        torch.cuda.synchronize()
        check(to_np(y), O.qlinear(x[0], w[0], s[0], b[0]), bound(O, x[0], s[0], b[0]), f"M={M}")


# ---- the widest MFMA tiles: 64 weight rows per workgroup (NT = 4) ----
# The host picks the most weight rows per workgroup (64, 32, 16) that still gives >= 512
# workgroups: n_layers * ceil(R / 64) * (m-tiles / MT) >= 512 selects 64.

@pytest.mark.parametrize("M", [40, 64])
def test_qlinear_mfma_in_proj_two_layers_64_row_tiles(O, gdn, dev, M):
    """The whole in_proj (R = 16480 rows, K = 5120) of two layers: 2 x 258 tiles of 64 rows =
    516 workgroups, so the 64-row form runs, with 3 (M = 40) and 4 (M = 64) m-tiles."""
    import torch
    log_case(f"qlinear (MFMA path, 64-row tiles) in_proj 4 segments x 2 layers, M={M}, K=5120")
    L, K = 2, 5120
    ns = [10240, 6144, 48, 48]
    mats, host, x = [], [], None
    for i, n in enumerate(ns):
        xi, w, s, b = quant_inputs(O, L, M, n, K, seed=600 + 10 * M + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w, s, b))
        host.append((w, s, b))
    ys = gdn.qlinear(mats, to_dev(x, dev), n_layers=L)
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        got = to_np(y)
        for l in range(L):
            check(got[l], O.qlinear_blocked(x[l], w[l], s[l], b[l]), bound(O, x[l], s[l], b[l]), f"segment {i} layer {l}")


@pytest.mark.parametrize("M,nseg", [(40, [300, 100]), (9, [700])])
def test_qlinear_mfma_eight_layers_whole_layers_per_xcd(O, gdn, dev, M, nseg):
    """8 layers in one launch: the workgroup ids are renumbered so each XCD runs whole layers
    (a layer's operand then reaches one L2); every layer and segment must still be right."""
    import torch
    log_case(f"qlinear (MFMA path) 8 layers, segments {nseg}, M={M}, K=1024")
    L, K = 8, 1024
    mats, host, x = [], [], None
    for i, n in enumerate(nseg):
        xi, w, s, b = quant_inputs(O, L, M, n, K, seed=1200 + 10 * M + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w, s, b))
        host.append((w, s, b))
    ys = gdn.qlinear(mats, to_dev(x, dev), n_layers=L)
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        got = to_np(y)
        for l in range(L):
            check(got[l], O.qlinear(x[l], w[l], s[l], b[l]), bound(O, x[l], s[l], b[l]), f"segment {i} layer {l}")


# ---- 256 weight rows per workgroup, the operand shared by its four waves through LDS ----
# One m group (M <= 64) and n_layers * ceil(R / 256) >= 512 select qgemm_ns_kernel: e.g.
# 8 layers of in_proj (65 workgroups a layer) or 26 of out_proj (20 a layer).

def sampled_rows(N, rng, n=768):
    """The first and last 256 rows and n - 512 others: every workgroup boundary case plus a
    spread, so the fp64 check stays short at K = 5120."""
    mid = rng.choice(np.arange(256, N - 256), size=n - 512, replace=False)
    return np.sort(np.concatenate([np.arange(256), np.arange(N - 256, N), mid]))


@pytest.mark.parametrize("M,K", [(5, 1024), (17, 1024), (40, 1024), (64, 1024), (40, 5120)])
def test_qlinear_mfma_in_proj_rows_shared_operand(O, gdn, dev, M, K):
    """8 layers of the in_proj row count (16,480 rows in its four matrices: segment bounds
    inside workgroups, the last workgroup partly past the rows), 520 workgroups of 256 rows,
    M from one to four m tiles; K = 1024 (8 steps of two groups, both scale and bias
    buffers, the repeated loads of the last steps) and K = 5120 (40 steps). At K = 5120 a
    sample of rows of every layer and segment is checked."""
    import torch
    log_case(f"qlinear (MFMA path, 256-row workgroups) in_proj 4 segments x 8 layers, M={M}, K={K}")
    L, nseg = 8, [10240, 6144, 48, 48]
    rng = np.random.default_rng(1500 + M + K)
    mats, host, x = [], [], None
    for i, n in enumerate(nseg):
        xi, w, s, b = quant_inputs(O, L, M, n, K, seed=1500 + 10 * M + K + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w, s, b))
        host.append((w, s, b))
    ys = gdn.qlinear(mats, to_dev(x, dev), n_layers=L)
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        got = to_np(y)
        n = w.shape[1]
        rows = sampled_rows(n, rng) if K > 1024 and n > 1024 else np.arange(n)
        for l in range(L):
            ws_, ss, bs = w[l][rows], s[l][rows], b[l][rows]
            check(got[l][:, rows], O.qlinear_blocked(x[l], ws_, ss, bs), bound(O, x[l], ss, bs),
                  f"segment {i} layer {l}")


def test_qlinear_mfma_out_proj_rows_shared_operand(O, gdn, dev):
    """out_proj(GatedRMSNorm(o, z)) over 26 layers (5,120 rows: 20 workgroups of 256 a
    layer, 520 in all), M = 40, K = 1024: the norm applied in the preparation kernel, the
    product in the operand-sharing kernel."""
    import torch
    log_case("qlinear (MFMA path, 256-row workgroups) out_proj with GatedRMSNorm x 26 layers, M=40, K=1024")
    L, M, K, N = 26, 40, 1024, 5120
    rng = np.random.default_rng(1600)
    o = (rng.standard_normal((L, M, K)) * 0.3).astype(np.float32)
    z = O.to_bf16(rng.standard_normal((L, M, K)).astype(np.float32))
    gamma = rng.uniform(0.5, 1.5, (L, 128)).astype(np.float32)
    _, w, s, b = quant_inputs(O, L, M, N, K, seed=1601)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w, s, b)],
                       norm=(to_dev(o, dev), to_dev(z, dev), to_dev(gamma, dev), 1e-6), n_layers=L)
    torch.cuda.synchronize()
    got = to_np(y)
    for l in range(L):
        xn = O.gated_rmsnorm(o[l].reshape(M * (K // 128), 128), z[l].reshape(M * (K // 128), 128),
                             gamma[l], 1e-6).reshape(M, K)
        ref = O.qlinear_blocked(xn, w[l], s[l], b[l])
        W = (np.abs(np.repeat(bf16_to_f32(s[l]), 64, axis=1)) * 15 + np.abs(np.repeat(bf16_to_f32(b[l]), 64, axis=1)))
        flip = 3 * 2.0 ** -8 * (np.abs(bf16_to_f32(xn)).max(axis=1, keepdims=True) * W.max(axis=1)[None, :])
        check(got[l], ref, bound(O, xn, s[l], b[l]) + flip, f"layer {l}")


def test_qlinear_mfma_512_rows(O, gdn, dev):
    """The most rows the quantized path takes (512 = 32 m-tiles in 8 groups of 4), N = 4096:
    64 tiles of 64 rows x 8 = 512 workgroups, so the 64-row form with 4 m-tiles runs."""
    import torch
    log_case("qlinear (MFMA path, 64-row tiles) M=512, N=4096, K=1024")
    M, N, K = 512, 4096, 1024
    x, w, s, b = quant_inputs(O, 1, M, N, K, seed=700)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])], to_dev(x[0], dev))
    torch.cuda.synchronize()
    check(to_np(y), O.qlinear_blocked(x[0], w[0], s[0], b[0]), bound(O, x[0], s[0], b[0]), "y")


# ---- prefill windows: more than 512 rows (the reference dequantizes and multiplies there,
# model.cpp:358-362, in windows of 1024 tokens, session.hpp:136; this path keeps the exact
# per-group arithmetic at every row count) ----

def test_qlinear_in_proj_prefill_window_1024_rows(O, gdn, dev):
    """A 1024-token window through the layer's four in_proj matrices (K = 5120; N reduced to
    1024 / 512 / 48 / 48 to keep the fp64 check short): 16 m groups of 64 rows, XCD-ordered."""
    import torch
    log_case("qlinear (MFMA path) in_proj 4 segments, M=1024, K=5120")
    M, K = 1024, 5120
    ns = [1024, 512, 48, 48]
    mats, host, x = [], [], None
    for i, n in enumerate(ns):
        xi, w, s, b = quant_inputs(O, 1, M, n, K, seed=800 + i)
        x = xi if x is None else x
        mats.append(dev_mat(gdn, dev, w[0], s[0], b[0]))
        host.append((w[0], s[0], b[0]))
    ys = gdn.qlinear(mats, to_dev(x[0], dev))
    torch.cuda.synchronize()
    for i, ((w, s, b), y) in enumerate(zip(host, ys)):
        check(to_np(y), O.qlinear_blocked(x[0], w, s, b), bound(O, x[0], s, b), f"segment {i}")


def test_qlinear_1024_rows_against_the_dequantize_path(O, gdn, dev):
    """At 512 rows and more the reference dequantizes each weight to bf16 and multiplies
    (model.cpp:358-362); this path keeps the exact per-group arithmetic. Measured here on a
    1024-token in_proj_qkv-shaped block (N reduced to 1024): the kernel's output against the
    oracle's emulation of the dequantize path (`qlinear_dequant_bf16`), and the emulation's
    own distance from the exact product -- relative to the output's largest magnitude, and
    held to the model's 1e-2."""
    import torch
    log_case("qlinear M=1024 against the reference's dequantize-then-matmul form, K=5120")
    M, N, K = 1024, 1024, 5120
    x, w, s, b = quant_inputs(O, 1, M, N, K, seed=830)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])], to_dev(x[0], dev))
    torch.cuda.synchronize()
    got = bf16_to_f32(to_np(y)).astype(np.float64)
    deq = O.qlinear_dequant_bf16(x[0], w[0], s[0], b[0])
    exact = O.qlinear_blocked(x[0], w[0], s[0], b[0])
    scale = np.abs(exact).max()
    d_kernel = np.abs(got - deq).max() / scale
    d_paths = np.abs(exact - deq).max() / scale
    d_exact = np.abs(got - exact).max() / scale
    print(f"  kernel vs dequantize path {d_kernel:.2e}, kernel vs exact {d_exact:.2e}, "
          f"dequantize path vs exact {d_paths:.2e} (max-abs / max |y|)", flush=True)
    assert d_kernel < 1e-2 and d_paths < 1e-2


def test_qlinear_out_proj_prefill_window_1024_rows(O, gdn, dev):
    """out_proj(GatedRMSNorm(o, z)) over a 1024-token window: K = 6144, N = 5120 (full size),
    the norm applied while the operand goes to the workspace; same tolerance as the M <= 512
    norm tests."""
    import torch
    log_case("qlinear (MFMA path) out_proj with GatedRMSNorm, M=1024, K=6144, N=5120")
    M, K, N = 1024, 6144, 5120
    rng = np.random.default_rng(901)
    o = (rng.standard_normal((M, K)) * 0.3).astype(np.float32)
    z = O.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    gamma = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    _, w, s, b = quant_inputs(O, 1, M, N, K, seed=902)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w[0], s[0], b[0])],
                       norm=(to_dev(o, dev), to_dev(z, dev), to_dev(gamma, dev), 1e-6))
    torch.cuda.synchronize()
    xn = O.gated_rmsnorm(o.reshape(M * 48, 128), z.reshape(M * 48, 128), gamma, 1e-6).reshape(M, K)
    ref = O.qlinear_blocked(xn, w[0], s[0], b[0])
    W = (np.abs(np.repeat(bf16_to_f32(s[0]), 64, axis=1)) * 15 + np.abs(np.repeat(bf16_to_f32(b[0]), 64, axis=1)))
    flip = 3 * 2.0 ** -8 * (np.abs(bf16_to_f32(xn)).max(axis=1, keepdims=True) * W.max(axis=1)[None, :])
    check(to_np(y), ref, bound(O, xn, s[0], b[0]) + flip, "y")


def test_qlinear_4096_rows_two_layers(O, gdn, dev):
    """The most rows (4096) on two stacked layers, K = 1024, N = 96: every m group of both
    layers, against the oracle."""
    import torch
    log_case("qlinear (MFMA path) M=4096, 2 layers, K=1024, N=96")
    L, M, N, K = 2, 4096, 96, 1024
    x, w, s, b = quant_inputs(O, L, M, N, K, seed=903)
    (y,) = gdn.qlinear([dev_mat(gdn, dev, w, s, b)], to_dev(x, dev), n_layers=L)
    torch.cuda.synchronize()
    got = to_np(y)
    for l in range(L):
        check(got[l], O.qlinear_blocked(x[l], w[l], s[l], b[l]), bound(O, x[l], s[l], b[l]), f"layer {l}")
