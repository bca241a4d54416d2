"""Pins the CPU oracle without trusting it: known-answer vectors for the
generator, independent implementations (torch's bf16 cast, fp64 libm, numpy fp64 matrix
algebra), closed forms and invariants of the recurrence, and the reference's own
criterion for the chunked form (equality with the per-token recurrence)."""
from __future__ import annotations

import math

import numpy as np
import pytest

D = 128


# ---------------------------------------------------------------- generator

def test_xoshiro256ss_known_answer(O):
    # Published output of xoshiro256** from state (1, 2, 3, 4) (the algorithm's
    # reference test sequence; also the first two values follow by hand:
    # rotl(2*5, 7)*9 = 11520, and s1 becomes 0 after one step).
    import ctypes
    s = (ctypes.c_uint64 * 4)(1, 2, 3, 4)
    got = [O.lib().gdno_xoshiro_next(s) for _ in range(10)]
    want = [11520, 0, 1509978240, 1215971899390074240, 1216172134540287360,
            607988272756665600, 16172922978634559625, 8476171486693032832,
            10595114339597558777, 2904607092377533576]
    assert got == want


def test_splitmix64_known_answer(O):
    import ctypes
    st = ctypes.c_uint64(0)
    # SplitMix64 from seed 0: first output 0xE220A8397B1DCDAF
    assert O.lib().gdno_splitmix64_next(ctypes.byref(st)) == 0xE220A8397B1DCDAF


def test_normal_generator_statistics(O):
    from scipy import stats
    x = O.normal(7, (200000,), 0.0, 1.0).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert stats.kstest(x, "norm").pvalue > 1e-3
    y = O.normal(7, (1000,), 0.5, 0.1)
    assert np.array_equal(y[:10], O.normal(7, (10,), 0.5, 0.1))  # reproducible prefix
    assert not np.array_equal(O.normal(8, (10,)), O.normal(7, (10,)))
    u = O.uniform(3, (100000,), -1.0, 1.0)
    assert u.min() >= -1.0 and u.max() < 1.0 and abs(u.mean()) < 0.01


# ---------------------------------------------------------------- bf16

def test_bf16_round_to_nearest_even_matches_torch(O):
    import torch
    x = np.concatenate([O.normal(1, (50000,), 0, 3), O.normal(2, (1000,), 0, 1e-30),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 0.0, -0.0,
                                  3.0e38, np.inf, -np.inf], np.float32)]).astype(np.float32)
    ours = O.to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    # ties go to even
    assert O.from_bf16(O.to_bf16(np.float32(1.0 + 2 ** -8)))[()] == 1.0
    assert O.from_bf16(O.to_bf16(np.float32(1.0 + 3 * 2 ** -8)))[()] == 1.0 + 2 ** -6


# ---------------------------------------------------------------- elementary functions

def _ulp_err(got: float, ref: float) -> float:
    return abs(got - ref) / float(np.spacing(np.float32(abs(ref))))


@pytest.mark.parametrize("name,ref,lo,hi,ulps", [
    ("expf", math.exp, -87.0, 88.0, 1.0),
    ("sigmoidf", lambda x: 1.0 / (1.0 + math.exp(-x)), -80.0, 40.0, 2.5),
    ("softplusf", lambda x: max(x, 0.0) + math.log1p(math.exp(-abs(x))), -60.0, 60.0, 4.0),
    ("log1pf", math.log1p, 0.0, 1.0, 3.0),
])
def test_elementary_functions_against_fp64(O, name, ref, lo, hi, ulps):
    xs = np.linspace(lo, hi, 20011).astype(np.float32)
    worst = max(_ulp_err(O.scalar(name, float(x)), ref(float(x))) for x in xs)
    assert worst <= ulps, (name, worst)


def test_elementary_closed_forms(O):
    assert O.scalar("sigmoidf", 0.0) == 0.5
    assert O.scalar("expf", 0.0) == 1.0
    assert _ulp_err(O.scalar("softplusf", 0.0), math.log(2.0)) <= 1
    assert O.scalar("softplusf", 50.0) == 50.0
    assert _ulp_err(O.scalar("softplusf", -50.0), math.exp(-50.0)) <= 2
    assert O.scalar("softplusf", float("inf")) == float("inf")
    assert O.scalar("softplusf", float("-inf")) == 0.0
    for x in np.linspace(-20, 20, 101).astype(np.float32):
        d = O.scalar("softplusf", float(x)) - O.scalar("softplusf", float(-x))
        assert abs(d - float(x)) <= 4 * float(np.spacing(np.float32(max(abs(x), 1.0))))
    assert O.scalar("expf", 89.0) == float("inf") and O.scalar("expf", -110.0) == 0.0


# ---------------------------------------------------------------- gates

def test_gates_closed_form(O):
    Hv = 48
    dt = O.normal(5, (Hv,), 0, 0.1)
    a_f = -dt  # a + dt_bias = 0 needs a bf16 a: use dt values that are bf16-exact
    dt = O.from_bf16(O.to_bf16(dt))
    a = O.to_bf16(-dt)
    b = O.to_bf16(np.zeros(Hv, np.float32))
    alpha, beta = O.gates(a, b, np.zeros(Hv, np.float32), dt)
    assert np.all(beta == 0.5)
    # alpha = exp(-exp(0) * softplus(0)) = exp(-ln 2) = 0.5 (to a few ulp)
    assert np.all(np.abs(alpha - 0.5) <= 4 * np.spacing(np.float32(0.5)))
    del a_f


def test_gates_against_fp64(O):
    Hv, rows = 48, 64
    a = O.to_bf16(O.normal(11, (rows, Hv)) * 4)
    b = O.to_bf16(O.normal(12, (rows, Hv)) * 4)
    A_log = O.uniform(13, (Hv,), -1, 1)
    dt = O.normal(14, (Hv,), 0, 0.1)
    alpha, beta = O.gates(a, b, A_log, dt)
    af, bf = O.from_bf16(a).astype(np.float64), O.from_bf16(b).astype(np.float64)
    sp = np.logaddexp(0.0, af + dt.astype(np.float64))
    alpha64 = np.exp(-np.exp(A_log.astype(np.float64)) * sp)
    beta64 = 1.0 / (1.0 + np.exp(-bf))
    assert np.max(np.abs(alpha - alpha64) / alpha64) < 3e-6
    assert np.max(np.abs(beta - beta64) / beta64) < 1e-6


# ---------------------------------------------------------------- front end

def test_l2norm_tree_sum_is_a_sum(O):
    sq = O.normal(3, (128,)) ** 2
    assert abs(O.sum128_tree(sq) - float(sq.astype(np.float64).sum())) < 1e-5 * sq.sum()
    ones = np.ones(128, np.float32)
    assert O.sum128_tree(ones) == 128.0


def _conv_inputs(O, B, L, Hk, Hv, seed):
    C = 2 * Hk * D + Hv * D
    x = O.to_bf16(O.normal(seed, (B, L, C)))
    cs = O.to_bf16(O.normal(seed + 1, (B, 3, C)))
    w = O.to_bf16(O.normal(seed + 2, (4, C), 0, 0.1))
    return x, cs, w


def test_frontend_norms_and_scale(O):
    x, cs, w = _conv_inputs(O, 2, 3, 2, 6, 100)
    q, k, v, xp = O.conv_frontend(x, cs, w, 2, 6)
    kn = np.linalg.norm(O.from_bf16(k).astype(np.float64), axis=-1)
    qn = np.linalg.norm(O.from_bf16(q).astype(np.float64), axis=-1)
    assert np.all(np.abs(kn - 1.0) < 2e-2)          # bf16 l2norm of a 128-vector
    assert np.all(np.abs(qn * math.sqrt(128) - 1.0) < 2e-2)
    assert xp.shape == (2, 6, x.shape[2])
    assert np.array_equal(xp[:, :3], cs) and np.array_equal(xp[:, 3:], x)


def test_frontend_silu_and_conv_against_fp64(O):
    """v channels are conv + silu only: compare with an fp64 evaluation (bf16 tolerance)."""
    B, L, Hk, Hv = 1, 5, 1, 3
    x, cs, w = _conv_inputs(O, B, L, Hk, Hv, 200)
    q, k, v, xp = O.conv_frontend(x, cs, w, Hk, Hv)
    xpf = O.from_bf16(xp).astype(np.float64)
    wf = O.from_bf16(w).astype(np.float64)
    y = np.stack([sum(xpf[:, t + j] * wf[j] for j in range(4)) for t in range(L)], axis=1)
    u = y / (1.0 + np.exp(-y))
    vref = u[..., 2 * Hk * D:].reshape(B, L, Hv, D)
    vf = O.from_bf16(v)
    assert np.max(np.abs(vf - vref)) <= 0.03 * np.max(np.abs(vref))
    # q,k: l2norm of the fp64 silu output
    qk = u[..., :2 * Hk * D].reshape(B, L, 2 * Hk, D)
    qk = qk / np.linalg.norm(qk, axis=-1, keepdims=True)
    assert np.max(np.abs(O.from_bf16(k)[:, :, 0] - qk[:, :, 1])) < 0.02
    assert np.max(np.abs(O.from_bf16(q)[:, :, 0] * math.sqrt(128) - qk[:, :, 0])) < 0.03


def test_frontend_delta_input_reproduces_taps(O):
    """A unit impulse at step 0 with a zero conv state: the conv output at step t is
    tap w[3-t] (the causal conv reverses the taps); v channels show silu of it."""
    B, L, Hk, Hv = 1, 4, 1, 3
    C = 2 * Hk * D + Hv * D
    x = np.zeros((B, L, C), np.uint16)
    x[0, 0, :] = O.to_bf16(np.ones(C, np.float32))
    w = O.to_bf16(O.normal(300, (4, C), 0, 0.5))
    _, _, v, _ = O.conv_frontend(x, None, w, Hk, Hv)
    wf = O.from_bf16(w).astype(np.float64)
    for t in range(L):
        y = wf[3 - t, 2 * Hk * D:]
        ref = y / (1.0 + np.exp(-y))
        assert np.max(np.abs(O.from_bf16(v)[0, t].reshape(-1) - ref)) <= 0.01 * np.max(np.abs(ref)) + 1e-6


def test_frontend_zero_state_and_streaming(O):
    B, L, Hk, Hv = 2, 7, 1, 3
    x, cs, w = _conv_inputs(O, B, L, Hk, Hv, 400)
    zero = np.zeros_like(cs)
    a = O.conv_frontend(x, None, w, Hk, Hv)
    b = O.conv_frontend(x, zero, w, Hk, Hv)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    # streaming in two segments equals one pass (segmented prefill principle)
    full = O.conv_frontend(x, cs, w, Hk, Hv)
    s1 = O.conv_frontend(np.ascontiguousarray(x[:, :3]), cs, w, Hk, Hv)
    s2 = O.conv_frontend(np.ascontiguousarray(x[:, 3:]), np.ascontiguousarray(s1[3][:, -3:]), w, Hk, Hv)
    for i in range(3):
        assert np.array_equal(np.concatenate([s1[i], s2[i]], axis=1), full[i])


# ---------------------------------------------------------------- recurrence

def _rand_step_inputs(O, B, L, Hk, Hv, seed, unit=True):
    q = O.normal(seed, (B, L, Hk, D))
    k = O.normal(seed + 1, (B, L, Hk, D))
    if unit:
        q = q / np.linalg.norm(q, axis=-1, keepdims=True) / math.sqrt(D)
        k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    v = O.normal(seed + 2, (B, L, Hv, D))
    al = O.uniform(seed + 3, (B, L, Hv), 0.85, 1.0)
    be = O.uniform(seed + 4, (B, L, Hv), 0.0, 1.0)
    S0 = O.normal(seed + 5, (B, Hv, D, D), 0, 0.1)
    return [np.ascontiguousarray(a, np.float32) for a in (q, k, v, al, be, S0)]


def _matrix_form_f64(q, k, v, al, be, S0, rep):
    """Independent fp64 formulation: S' = a S (I - b k k^T) + b v k^T, o = S' q, with the
    state (Dv, Dk) as matrices (numpy matmul), per (batch, head)."""
    B, L, Hk, _ = q.shape
    Hv = v.shape[2]
    S = S0.astype(np.float64).copy()
    o = np.zeros((B, L, Hv, D))
    I = np.eye(D)
    for b in range(B):
        for h in range(Hv):
            for t in range(L):
                kk = k[b, t, h // rep].astype(np.float64)
                qq = q[b, t, h // rep].astype(np.float64)
                vv = v[b, t, h].astype(np.float64)
                P = I - be[b, t, h] * np.outer(kk, kk)
                S[b, h] = al[b, t, h] * (S[b, h] @ P) + be[b, t, h] * np.outer(vv, kk)
                o[b, t, h] = S[b, h] @ qq
    return o, S


def test_recurrence_matches_matrix_formulation(O):
    q, k, v, al, be, S0 = _rand_step_inputs(O, 2, 5, 2, 6, 500)
    o32, S32 = O.recurrent(q, k, v, al, be, S0)
    o64, S64 = O.recurrent_f64(q, k, v, al, be, S0)
    om, Sm = _matrix_form_f64(q, k, v, al, be, S0, rep=3)
    assert O.rel_err(o64, om) < 1e-12 and O.rel_err(S64, Sm) < 1e-12
    assert O.rel_err(o32, om) < 2e-6 and O.rel_err(S32, Sm) < 2e-6


def test_recurrence_zero_state_closed_form(O):
    q, k, v, al, be, _ = _rand_step_inputs(O, 1, 1, 2, 6, 600)
    o, S = O.recurrent(q, k, v, al, be, None)
    for h in range(6):
        kk, qq = k[0, 0, h // 3].astype(np.float64), q[0, 0, h // 3].astype(np.float64)
        Sref = be[0, 0, h] * np.outer(v[0, 0, h], kk)
        assert np.max(np.abs(S[0, h] - Sref)) < 1e-6
        assert np.max(np.abs(o[0, 0, h] - be[0, 0, h] * v[0, 0, h] * (kk @ qq))) < 1e-6


def test_recurrence_beta_zero_decays(O):
    q, k, v, al, be, S0 = _rand_step_inputs(O, 1, 1, 2, 6, 700)
    be[:] = 0.0
    o, S = O.recurrent(q, k, v, al, be, S0)
    for h in range(6):
        assert np.array_equal(S[0, h], (al[0, 0, h] * S0[0, h]).astype(np.float32))
        assert np.max(np.abs(o[0, 0, h] - (al[0, 0, h] * S0[0, h].astype(np.float64)) @ q[0, 0, h // 3])) < 1e-6


def test_recurrence_delta_rule_write_invariant(O):
    """For unit k: S'k = a(1-b) S k + b v; with a = b = 1 the state stores v under k."""
    q, k, v, al, be, S0 = _rand_step_inputs(O, 1, 1, 2, 6, 800)
    o, S = O.recurrent(q, k, v, al, be, S0)
    for h in range(6):
        kk = k[0, 0, h // 3].astype(np.float64)
        lhs = S[0, h].astype(np.float64) @ kk
        rhs = al[0, 0, h] * (1 - be[0, 0, h]) * (S0[0, h].astype(np.float64) @ kk) + be[0, 0, h] * v[0, 0, h]
        assert np.max(np.abs(lhs - rhs)) < 1e-5
    al[:] = 1.0
    be[:] = 1.0
    o, S = O.recurrent(q, k, v, al, be, S0)
    for h in range(6):
        assert np.max(np.abs(S[0, h].astype(np.float64) @ k[0, 0, h // 3] - v[0, 0, h])) < 1e-5


def test_recurrence_readout_linear_in_q(O):
    q, k, v, al, be, S0 = _rand_step_inputs(O, 1, 3, 1, 3, 900)
    q2 = O.normal(901, q.shape) * 0.1
    o1, _ = O.recurrent(q, k, v, al, be, S0)
    o2, _ = O.recurrent(q2, k, v, al, be, S0)
    o3, _ = O.recurrent(q + q2, k, v, al, be, S0)
    assert O.rel_err(o3, o1 + o2) < 1e-5


def test_recurrence_collect_and_materialized(O):
    q, k, v, al, be, S0 = _rand_step_inputs(O, 2, 4, 2, 6, 1000)
    o, S, states = O.recurrent(q, k, v, al, be, S0, collect=True)
    assert np.array_equal(states[:, :, -1], S)
    for t in range(4):
        ot, St = O.recurrent(q[:, :t + 1], k[:, :t + 1], v[:, :t + 1], al[:, :t + 1],
                             be[:, :t + 1], S0)
        assert np.array_equal(states[:, :, t], St) and np.array_equal(o[:, :t + 1], ot)
    om, Sm, stm = O.recurrent(q, k, v, al, be, S0, collect=True, materialize=True, threads=3)
    assert np.array_equal(om, o) and np.array_equal(Sm, S) and np.array_equal(stm, states)


def test_gqa_head_map_is_repeat_interleave(O):
    """v-head h reads k-head h // rep: with head-distinct k and a zero state, o of v-head h
    is b v (k_{h//rep} . q_{h//rep})."""
    B, L, Hk, Hv = 1, 1, 4, 12
    q, k, v, al, be, _ = _rand_step_inputs(O, B, L, Hk, Hv, 1100)
    o, _ = O.recurrent(q, k, v, al, be, None)
    for h in range(Hv):
        g = h // 3
        want = be[0, 0, h] * v[0, 0, h] * float(k[0, 0, g].astype(np.float64) @ q[0, 0, g])
        assert np.max(np.abs(o[0, 0, h] - want)) < 1e-6
        if g != (h % Hk):  # a tile-order map would read another head
            wrong = be[0, 0, h] * v[0, 0, h] * float(k[0, 0, h % Hk] @ q[0, 0, h % Hk])
            assert np.max(np.abs(o[0, 0, h] - wrong)) > 1e-4


# ---------------------------------------------------------------- chunked form

@pytest.mark.parametrize("L", [1, 5, 16, 63, 64, 65, 130, 200])
def test_chunked_equals_per_token(O, L):
    """The reference's criterion (BUILD_LOG.md:314-315: rel-err <= 1.8e-6 in fp32)."""
    q, k, v, al, be, S0 = _rand_step_inputs(O, 1, L, 1, 3, 1200 + L)
    oc, Sc = O.chunked(q, k, v, al, be, S0)
    os_, Ss = O.recurrent(q, k, v, al, be, S0)
    assert O.rel_err(oc, os_) < 1e-5 and O.rel_err(Sc, Ss) < 1e-5


def test_chunked_chunk_of_one_is_sequential(O):
    q, k, v, al, be, S0 = _rand_step_inputs(O, 1, 9, 1, 3, 1300)
    oc, Sc = O.chunked(q, k, v, al, be, S0, C=1)
    os_, Ss = O.recurrent(q, k, v, al, be, S0)
    assert O.rel_err(oc, os_) < 1e-6 and O.rel_err(Sc, Ss) < 1e-6


def test_chunked_padding_is_a_no_op(O):
    """Appending steps with alpha=1, beta=0 and q=k=v=0 leaves the state unchanged."""
    q, k, v, al, be, S0 = _rand_step_inputs(O, 1, 70, 1, 3, 1400)
    pad = lambda a, val: np.concatenate([a, np.full((1, 10) + a.shape[2:], val, a.dtype)], 1)  # noqa: E731
    o1, S1 = O.chunked(q, k, v, al, be, S0)
    o2, S2 = O.chunked(pad(q, 0), pad(k, 0), pad(v, 0), pad(al, 1.0), pad(be, 0.0), S0)
    assert np.array_equal(S1, S2) and np.array_equal(o1, o2[:, :70])


def test_chunked_zero_initial_state(O):
    q, k, v, al, be, _ = _rand_step_inputs(O, 1, 100, 1, 3, 1500)
    oc, Sc = O.chunked(q, k, v, al, be, None)
    os_, Ss = O.recurrent(q, k, v, al, be, None)
    assert O.rel_err(oc, os_) < 1e-5 and O.rel_err(Sc, Ss) < 1e-5


# ---------------------------------------------------------------- commit

def test_commit_semantics(O):
    B, T, Hk, Hv = 1, 5, 1, 3
    C = 2 * Hk * D + Hv * D
    q, k, v, al, be, S0 = _rand_step_inputs(O, B, T, Hk, Hv, 1600)
    o, S, states = O.recurrent(q, k, v, al, be, S0, collect=True)
    x = O.to_bf16(O.normal(1601, (B, T, C)))
    cs = O.to_bf16(O.normal(1602, (B, 3, C)))
    xp = np.concatenate([cs, x], axis=1)
    for n in range(T + 1):
        Sn, conv = O.commit(n, states, S0, xp)
        assert np.array_equal(Sn, S0 if n == 0 else states[:, :, n - 1])
        assert np.array_equal(conv, xp[:, n:n + 3])
        if n > 0:  # equals running n steps from S_prev
            _, Sr = O.recurrent(q[:, :n], k[:, :n], v[:, :n], al[:, :n], be[:, :n], S0)
            assert np.array_equal(Sn, Sr)
    with pytest.raises(ValueError):
        O.commit(T + 1, states, S0, xp)
    with pytest.raises(ValueError):
        O.commit(-1, states, S0, xp)


# ---------------------------------------------------------------- quantized linear / norm

def _unpack_np(w):
    """Independent unpacking of the 4-bit layout with numpy bit ops: value i of a word in
    nibble i, low nibble first (python/mlp_kernel.py:54-56)."""
    N, W8 = w.shape
    sh = (4 * np.arange(8, dtype=np.uint32))
    return ((w[:, :, None] >> sh) & 0xF).reshape(N, W8 * 8).astype(np.float64)


def _qlin_inputs(O, M, N, K, seed):
    rng = np.random.default_rng(seed)
    x = O.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = O.to_bf16(rng.uniform(0.005, 0.05, (N, K // 64)).astype(np.float32))
    b = O.to_bf16(rng.uniform(-0.2, 0.2, (N, K // 64)).astype(np.float32))
    return x, w, s, b


def test_qlinear_matches_numpy_dequantize(O):
    x, w, s, b = _qlin_inputs(O, 3, 37, 256, 5)
    W = (_unpack_np(w) * np.repeat(O.from_bf16(s).astype(np.float64), 64, axis=1)
         + np.repeat(O.from_bf16(b).astype(np.float64), 64, axis=1))
    ref = O.from_bf16(x).astype(np.float64) @ W.T
    assert np.abs(O.qlinear(x, w, s, b) - ref).max() <= 1e-12 * np.abs(ref).max()


def test_qlinear_blocked_equals_qlinear(O):
    """The blocked numpy form (used for large GPU checks) equals the C oracle, with row blocks
    that split the matrix unevenly."""
    x, w, s, b = _qlin_inputs(O, 5, 300, 1024, 6)
    ref = O.qlinear(x, w, s, b)
    got = O.qlinear_blocked(x, w, s, b, rows=128)
    assert np.abs(got - ref).max() <= 1e-12 * np.abs(ref).max()


def test_qlinear_dequant_bf16_pins(O):
    """The reference's dequantize-then-matmul form (512 rows and more): where every weight
    s q + b is exact in bf16 (scales a power of two, biases on a coarse grid) it equals the
    exact product; with scales that are not, it differs from it by exactly the bf16 rounding
    of each weight (checked against weights rounded independently here), and the difference
    is a small fraction of the output."""
    x, w, s, b = _qlin_inputs(O, 3, 40, 256, 7)
    s_exact = O.to_bf16(np.full(s.shape, 0.25, np.float32))
    b_exact = O.to_bf16(np.round(O.from_bf16(b) * 4) / 4)
    ref = O.qlinear(x, w, s_exact, b_exact)
    assert np.abs(O.qlinear_dequant_bf16(x, w, s_exact, b_exact, rows=100) - ref).max() <= 1e-12 * np.abs(ref).max()
    # general scales: the weights rounded to bf16 one by one (round to nearest even on the
    # fp32 value, as torch rounds), then an fp64 product
    q = _unpack_np(w)
    Wd = (q * np.repeat(O.from_bf16(s).astype(np.float64), 64, axis=1)
          + np.repeat(O.from_bf16(b).astype(np.float64), 64, axis=1))
    import torch
    Wb = torch.from_numpy(Wd.astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()
    want = O.from_bf16(x).astype(np.float64) @ Wb.T
    got = O.qlinear_dequant_bf16(x, w, s, b, rows=100)
    assert np.abs(got - want).max() <= 1e-12 * np.abs(want).max()
    exact = O.qlinear(x, w, s, b)
    gap = np.abs(got - exact).max() / np.abs(exact).max()
    assert 0 < gap < 2 ** -7


def test_qlinear_nibble_order_known_answers(O):
    """A single nonzero nibble at value position i of word j selects x[8j + i]; scale 1,
    bias 0; an all-zero w with bias b gives b * sum(x) per group."""
    K, N = 128, 16
    x = O.to_bf16(np.arange(1, K + 1, dtype=np.float32) / 64)
    xf = O.from_bf16(x).astype(np.float64)
    w = np.zeros((N, K // 8), np.uint32)
    for n in range(N):
        j, i = n % (K // 8), n % 8
        w[n, j] = np.uint32(3) << np.uint32(4 * i)
    one = O.to_bf16(np.ones((N, K // 64), np.float32))
    zero = O.to_bf16(np.zeros((N, K // 64), np.float32))
    y = O.qlinear(x[None], w, one, zero)[0]
    for n in range(N):
        j, i = n % (K // 8), n % 8
        assert y[n] == 3 * xf[8 * j + i]
    half = O.to_bf16(np.full((N, K // 64), 0.5, np.float32))
    y = O.qlinear(x[None], np.zeros_like(w), one, half)[0]
    assert np.allclose(y, 0.5 * xf.sum())


def test_gated_rmsnorm_closed_forms_and_fp64(O):
    rng = np.random.default_rng(9)
    o = rng.standard_normal((6, 128)).astype(np.float32)
    z = O.to_bf16(rng.standard_normal((6, 128)).astype(np.float32))
    g = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    out = O.from_bf16(O.gated_rmsnorm(o, z, g, 1e-6)).astype(np.float64)
    od, zd = o.astype(np.float64), O.from_bf16(z).astype(np.float64)
    ref = od / np.sqrt((od ** 2).mean(-1, keepdims=True) + 1e-6) * g * (zd / (1 + np.exp(-zd)))
    assert np.all(np.abs(out - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-7)
    # silu(0) = 0 gates everything off
    assert np.all(O.gated_rmsnorm(o, O.to_bf16(np.zeros_like(o)), g, 1e-6) & 0x7FFF == 0)
    # scale invariance of the norm (eps aside): o and 1000 o give the same output
    a = O.gated_rmsnorm(o, z, g, 0.0)
    bb = O.gated_rmsnorm(o * 1024.0, z, g, 0.0)
    assert np.array_equal(a, bb)
    # a constant row c normalises to sign(c) gamma
    c = np.full((1, 128), -3.0, np.float32)
    one = O.to_bf16(np.full((1, 128), 20.0, np.float32))   # silu(20) rounds to 20
    r = O.from_bf16(O.gated_rmsnorm(c, one, g, 0.0))[0]
    expect = O.from_bf16(O.to_bf16((-g * (20.0 / (1 + np.exp(-20.0)))).astype(np.float32)))
    assert np.allclose(r, expect, rtol=2 ** -8)
