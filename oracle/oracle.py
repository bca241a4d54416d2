"""ctypes front for the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

The oracle restates the reference's unfused MLX op sequence for the gated-delta
path (citations in gdn_oracle.h / gdn_oracle.c). Only tests/, the smoke check and
bench.py's CPU-baseline leg import this module; the product never does.

bf16 arrays are numpy uint16 bit patterns. Shapes follow gdn_oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
D = 128
KCONV = 4

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i64 = ctypes.c_int64
_int = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    L.gdno_splitmix64_next.argtypes = [_u64p]
    L.gdno_splitmix64_next.restype = ctypes.c_uint64
    L.gdno_xoshiro_seed.argtypes = [_u64p, ctypes.c_uint64]
    L.gdno_xoshiro_next.argtypes = [_u64p]
    L.gdno_xoshiro_next.restype = ctypes.c_uint64
    L.gdno_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _f32p, _i64]
    L.gdno_fill_uniform.argtypes = [ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _f32p, _i64]
    L.gdno_f32_to_bf16.argtypes = [ctypes.c_float]
    L.gdno_f32_to_bf16.restype = ctypes.c_uint16
    L.gdno_round_bf16.argtypes = [_f32p, _u16p, _i64]
    L.gdno_widen_bf16.argtypes = [_u16p, _f32p, _i64]
    for name in ("gdno_expf", "gdno_logf", "gdno_log1pf", "gdno_sigmoidf", "gdno_softplusf",
                 "gdno_rsqrtf"):
        getattr(L, name).argtypes = [ctypes.c_float]
        getattr(L, name).restype = ctypes.c_float
    L.gdno_sum128_tree.argtypes = [_f32p]
    L.gdno_sum128_tree.restype = ctypes.c_float
    L.gdno_gates.argtypes = [_i64, _int, _u16p, _u16p, _f32p, _f32p, _f32p, _f32p]
    L.gdno_conv_frontend.argtypes = [_int, _int, _int, _int, _u16p, _u16p, _u16p, _u16p,
                                     _u16p, _u16p, _u16p]
    L.gdno_recurrent_f32.argtypes = [_int, _int, _int, _int, _f32p, _f32p, _f32p, _f32p,
                                     _f32p, _f32p, _f32p, _f32p, _f32p, _int, _int]
    L.gdno_recurrent_f64.argtypes = [_int, _int, _int, _int, _f32p, _f32p, _f32p, _f32p,
                                     _f32p, _f32p, _f64p, _f64p, _int]
    L.gdno_chunked_f32.argtypes = [_int, _int, _int, _int, _int, _f32p, _f32p, _f32p, _f32p,
                                   _f32p, _f32p, _f32p, _f32p, _int]
    L.gdno_commit.argtypes = [_int, _int, _int, _int, _int, _f32p, _f32p, _u16p, _f32p, _u16p]
    L.gdno_qlinear_f64.argtypes = [_int, _int, _int, _u16p, _u32p, _u16p, _u16p, _f64p]
    L.gdno_gated_rmsnorm.argtypes = [_i64, _int, _f32p, _u16p, _f32p, ctypes.c_float, _u16p]
    L.gdno_commit.restype = _int


def _p(a: np.ndarray | None, ct):
    if a is None:
        return ctypes.cast(None, ct)
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ct)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


# --------------------------------------------------------------------------
# generator and bf16

def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().gdno_fill_normal(seed, mean, std, _p(out, _f32p), out.size)
    return out.reshape(shape)


def uniform(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().gdno_fill_uniform(seed, lo, hi, _p(out, _f32p), out.size)
    return out.reshape(shape)


def to_bf16(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().gdno_round_bf16(_p(a, _f32p), _p(out, _u16p), a.size)
    return out


def from_bf16(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    lib().gdno_widen_bf16(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def scalar(name: str, x: float) -> float:
    return float(getattr(lib(), "gdno_" + name)(x))


def sum128_tree(sq) -> float:
    sq = _f32(sq)
    assert sq.size == 128
    return float(lib().gdno_sum128_tree(_p(sq, _f32p)))


# --------------------------------------------------------------------------
# op sequence

def gates(a_bf16, b_bf16, A_log, dt_bias):
    a_bf16, b_bf16 = _u16(a_bf16), _u16(b_bf16)
    A_log, dt_bias = _f32(A_log), _f32(dt_bias)
    Hv = A_log.size
    rows = a_bf16.size // Hv
    alpha = np.empty(a_bf16.shape, np.float32)
    beta = np.empty(a_bf16.shape, np.float32)
    lib().gdno_gates(rows, Hv, _p(a_bf16, _u16p), _p(b_bf16, _u16p), _p(A_log, _f32p),
                     _p(dt_bias, _f32p), _p(alpha, _f32p), _p(beta, _f32p))
    return alpha, beta


def conv_frontend(x_bf16, conv_state_bf16, w_bf16, Hk: int, Hv: int):
    """x (B,L,C), conv_state (B,3,C) or None, w (4,C) -> q,k (B,L,Hk,128), v (B,L,Hv,128), xp."""
    x = _u16(x_bf16)
    B, L, C = x.shape
    assert C == 2 * Hk * D + Hv * D
    cs = None if conv_state_bf16 is None else _u16(conv_state_bf16)
    w = _u16(w_bf16)
    q = np.empty((B, L, Hk, D), np.uint16)
    k = np.empty((B, L, Hk, D), np.uint16)
    v = np.empty((B, L, Hv, D), np.uint16)
    xp = np.empty((B, L + KCONV - 1, C), np.uint16)
    lib().gdno_conv_frontend(B, L, Hk, Hv, _p(x, _u16p), _p(cs, _u16p), _p(w, _u16p),
                             _p(q, _u16p), _p(k, _u16p), _p(v, _u16p), _p(xp, _u16p))
    return q, k, v, xp


def recurrent(q, k, v, alpha, beta, S_in=None, collect=False, materialize=False, threads=0):
    """fp32 restatement of delta::run_reference. q,k (B,L,Hk,128), v (B,L,Hv,128)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    alpha, beta = _f32(alpha), _f32(beta)
    B, L, Hk, _ = q.shape
    Hv = v.shape[2]
    S_out = np.empty((B, Hv, D, D), np.float32)
    o = np.empty((B, L, Hv, D), np.float32)
    states = np.empty((B, Hv, L, D, D), np.float32) if collect else None
    S_in = None if S_in is None else _f32(S_in)
    lib().gdno_recurrent_f32(B, L, Hk, Hv, _p(q, _f32p), _p(k, _f32p), _p(v, _f32p),
                             _p(alpha, _f32p), _p(beta, _f32p), _p(S_in, _f32p),
                             _p(S_out, _f32p), _p(o, _f32p), _p(states, _f32p),
                             int(bool(materialize)), threads)
    return (o, S_out, states) if collect else (o, S_out)


def recurrent_f64(q, k, v, alpha, beta, S_in=None, threads=0):
    q, k, v = _f32(q), _f32(k), _f32(v)
    alpha, beta = _f32(alpha), _f32(beta)
    B, L, Hk, _ = q.shape
    Hv = v.shape[2]
    S_out = np.empty((B, Hv, D, D), np.float64)
    o = np.empty((B, L, Hv, D), np.float64)
    S_in = None if S_in is None else _f32(S_in)
    lib().gdno_recurrent_f64(B, L, Hk, Hv, _p(q, _f32p), _p(k, _f32p), _p(v, _f32p),
                             _p(alpha, _f32p), _p(beta, _f32p), _p(S_in, _f32p),
                             _p(S_out, _f64p), _p(o, _f64p), threads)
    return o, S_out


def chunked(q, k, v, alpha, beta, S_in=None, C=64, threads=0):
    q, k, v = _f32(q), _f32(k), _f32(v)
    alpha, beta = _f32(alpha), _f32(beta)
    B, L, Hk, _ = q.shape
    Hv = v.shape[2]
    S_out = np.empty((B, Hv, D, D), np.float32)
    o = np.empty((B, L, Hv, D), np.float32)
    S_in = None if S_in is None else _f32(S_in)
    lib().gdno_chunked_f32(B, L, Hk, Hv, C, _p(q, _f32p), _p(k, _f32p), _p(v, _f32p),
                           _p(alpha, _f32p), _p(beta, _f32p), _p(S_in, _f32p),
                           _p(S_out, _f32p), _p(o, _f32p), threads)
    return o, S_out


def commit(n: int, states, S_prev, xp_bf16):
    """DeltaCache::commit(n): returns (state, conv) or raises ValueError like the reference."""
    states, S_prev, xp = _f32(states), _f32(S_prev), _u16(xp_bf16)
    B, Hv, T = states.shape[:3]
    C = xp.shape[2]
    S_dst = np.empty((B, Hv, D, D), np.float32)
    conv = np.empty((B, KCONV - 1, C), np.uint16)
    rc = lib().gdno_commit(B, T, Hv, C, n, _p(states, _f32p), _p(S_prev, _f32p), _p(xp, _u16p),
                           _p(S_dst, _f32p), _p(conv, _u16p))
    if rc != 0:
        raise ValueError("DeltaCache::commit out of range")
    return S_dst, conv


def qlinear(x_bf16, w_u32, scales_bf16, biases_bf16):
    """Linear::operator(), quantized branch (mx::quantized_matmul, 4-bit, group 64):
    x (M, K) bf16 bits, w (N, K/8) uint32, scales/biases (N, K/64) bf16 bits -> (M, N) fp64."""
    x, s, b = _u16(x_bf16), _u16(scales_bf16), _u16(biases_bf16)
    w = np.ascontiguousarray(w_u32, dtype=np.uint32)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape == (N, K // 8) and s.shape == (N, K // 64) and b.shape == (N, K // 64)
    y = np.empty((M, N), np.float64)
    lib().gdno_qlinear_f64(M, N, K, _p(x, _u16p), _p(w, _u32p), _p(s, _u16p), _p(b, _u16p),
                           _p(y, _f64p))
    return y


def qlinear_dequant_bf16(x_bf16, w_u32, scales_bf16, biases_bf16, rows: int = 2048):
    """The reference's Linear at 512 rows and more (cpp/src/model.cpp:358-362, kDequantRows
    = 512 in cpp/src/model.hpp:137): mx::dequantize to bf16 -- each weight s q + b rounded
    once to bf16 (MLX evaluates bf16 arithmetic in fp32 and rounds the result) -- then the
    bf16 matmul, modelled with an fp64 accumulation (MLX's order is not pinned) -> (M, N)
    fp64, before the output's bf16 rounding. Differs from qlinear by one bf16 rounding of
    every weight; tests/test_oracle.py pins it where those roundings are exact."""
    x = from_bf16(np.ascontiguousarray(x_bf16, np.uint16)).astype(np.float64)
    w = np.ascontiguousarray(w_u32, dtype=np.uint32)
    s = from_bf16(np.ascontiguousarray(scales_bf16, np.uint16)).astype(np.float64)
    b = from_bf16(np.ascontiguousarray(biases_bf16, np.uint16)).astype(np.float64)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape == (N, K // 8) and s.shape == (N, K // 64) and b.shape == (N, K // 64)
    shifts = 4 * np.arange(8, dtype=np.uint32)
    y = np.empty((M, N), np.float64)
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        q = ((w[r0:r1, :, None] >> shifts) & 0xF).reshape(r1 - r0, K).astype(np.float64)
        Wd = (q.reshape(r1 - r0, K // 64, 64) * s[r0:r1, :, None] + b[r0:r1, :, None]).reshape(r1 - r0, K)
        Wb = from_bf16(to_bf16(Wd.astype(np.float32))).astype(np.float64)
        y[:, r0:r1] = x @ Wb.T
    return y


def qlinear_blocked(x_bf16, w_u32, scales_bf16, biases_bf16, rows: int = 2048):
    """The same product as qlinear for large shapes: W dequantized to fp64 with numpy bit
    ops (value i of a word in nibble i, python/mlp_kernel.py:54-56) a block of rows at a
    time, then an fp64 matrix product -> (M, N) fp64. Equal to qlinear up to fp64 summation
    order (tests/test_oracle.py pins it)."""
    x = from_bf16(np.ascontiguousarray(x_bf16, np.uint16)).astype(np.float64)
    w = np.ascontiguousarray(w_u32, dtype=np.uint32)
    s = from_bf16(np.ascontiguousarray(scales_bf16, np.uint16)).astype(np.float64)
    b = from_bf16(np.ascontiguousarray(biases_bf16, np.uint16)).astype(np.float64)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape == (N, K // 8) and s.shape == (N, K // 64) and b.shape == (N, K // 64)
    shifts = 4 * np.arange(8, dtype=np.uint32)
    y = np.empty((M, N), np.float64)
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        q = ((w[r0:r1, :, None] >> shifts) & 0xF).reshape(r1 - r0, K).astype(np.float64)
        Wd = (q.reshape(r1 - r0, K // 64, 64) * s[r0:r1, :, None] + b[r0:r1, :, None]).reshape(r1 - r0, K)
        y[:, r0:r1] = x @ Wd.T
    return y


def gated_rmsnorm(o, z_bf16, gamma, eps: float = 1e-6):
    """GatedRMSNorm: rows of o (..., D) fp32, z bf16 bits, gamma (D) fp32 -> bf16 bits."""
    o, z, g = _f32(o), _u16(z_bf16), _f32(gamma)
    D = o.shape[-1]
    rows = o.size // D
    out = np.empty(o.shape, np.uint16)
    lib().gdno_gated_rmsnorm(rows, D, _p(o, _f32p), _p(z, _u16p), _p(g, _f32p), eps,
                             _p(out, _u16p))
    return out


# --------------------------------------------------------------------------
# synthetic inputs: seed = 1000*config + 17*layer + stream

STREAM = dict(q=0, k=1, v=2, a=3, b=4, A_log=5, dt_bias=6, state=7, conv_w=8, conv_state=9)


def seed_of(config: int, layer: int, stream: str) -> int:
    return 1000 * config + 17 * layer + STREAM[stream]


def l2norm_rows_bf16(x: np.ndarray) -> np.ndarray:
    """Normalise the last axis in fp64 and round to bf16 (input generation only)."""
    x64 = x.astype(np.float64)
    n = np.sqrt((x64 * x64).sum(-1, keepdims=True))
    return to_bf16((x64 / n).astype(np.float32))


@dataclass
class LayerInputs:
    q: np.ndarray | None        # (B,L,Hk,128) bf16, qkv front end
    k: np.ndarray | None
    v: np.ndarray | None        # (B,L,Hv,128) bf16
    x: np.ndarray | None        # (B,L,C) bf16, conv front end
    conv_w: np.ndarray | None   # (4,C) bf16
    conv_state: np.ndarray | None  # (B,3,C) bf16 or None (zeros)
    a: np.ndarray               # (B,L,Hv) bf16
    b: np.ndarray
    A_log: np.ndarray           # (Hv,) fp32
    dt_bias: np.ndarray
    state: np.ndarray | None    # (B,Hv,128,128) fp32 or None (zeros)


def make_inputs(config: int, layer: int, B: int, L: int, Hk: int = 16, Hv: int = 48,
                conv: bool = False, conv_state: bool = True, zero_state: bool = False,
                state_std: float = 0.02) -> LayerInputs:
    """Seeded inputs with the distributions of the benchmark configurations."""
    s = lambda name: seed_of(config, layer, name)  # noqa: E731
    q = l2norm_rows_bf16(normal(s("q"), (B, L, Hk, D)))
    k = l2norm_rows_bf16(normal(s("k"), (B, L, Hk, D)))
    v = to_bf16(normal(s("v"), (B, L, Hv, D)))
    a = to_bf16(normal(s("a"), (B, L, Hv)))
    b = to_bf16(normal(s("b"), (B, L, Hv)))
    A_log = uniform(s("A_log"), (Hv,), -1.0, 1.0)
    dt_bias = normal(s("dt_bias"), (Hv,), 0.0, 0.1)
    state = None if zero_state else normal(s("state"), (B, Hv, D, D), 0.0, state_std)
    if not conv:
        return LayerInputs(q, k, v, None, None, None, a, b, A_log, dt_bias, state)
    C = 2 * Hk * D + Hv * D
    x = np.concatenate([q.reshape(B, L, Hk * D), k.reshape(B, L, Hk * D),
                        v.reshape(B, L, Hv * D)], axis=-1)
    w = to_bf16(normal(s("conv_w"), (KCONV, C), 0.0, 0.1))
    cs = to_bf16(normal(s("conv_state"), (B, KCONV - 1, C))) if conv_state else None
    return LayerInputs(None, None, None, np.ascontiguousarray(x), w, cs, a, b, A_log, dt_bias,
                       state)


def reference_layer(inp: LayerInputs, collect: bool = False, materialize: bool = False,
                    threads: int = 0):
    """The reference's per-layer sequence (model.cpp:582-624): front end, gates,
    run_reference. Returns dict with o (fp32), state, states, xp, and the fp32 q,k,v."""
    Hv = inp.A_log.size
    if inp.x is not None:
        Hk = (inp.x.shape[2] - Hv * D) // (2 * D)
        qb, kb, vb, xp = conv_frontend(inp.x, inp.conv_state, inp.conv_w, Hk, Hv)
    else:
        qb, kb, vb, xp = inp.q, inp.k, inp.v, None
    q, k, v = from_bf16(qb), from_bf16(kb), from_bf16(vb)
    alpha, beta = gates(inp.a, inp.b, inp.A_log, inp.dt_bias)
    res = recurrent(q, k, v, alpha, beta, inp.state, collect=collect, materialize=materialize,
                    threads=threads)
    out = dict(o=res[0], state=res[1], states=res[2] if collect else None, xp=xp, q=q, k=k,
               v=v, alpha=alpha, beta=beta)
    return out


def rel_err(a, b) -> float:
    """max|a-b| / max|b|, the reference's measure (cpp/src/tests.cpp:38-45)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.abs(b).max() if b.size else 0.0
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0)) if b.size else 0.0


def max_abs(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max()) if b.size else 0.0
