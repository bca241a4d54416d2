"""GPU parity of the chunked prefill (chunk 64, bf16 MFMA) against the oracle's
token-by-token recurrence -- the reference's own criterion for its chunked form
(python/test_model.py:138-156, BUILD_LOG.md:314-315).

Tolerance: outputs within 1e-2 of the token-by-token result in the reference's measure
max|a-b|/max|b| (the task statement's bound for chunked prefill); the bf16 output rounding
(up to 2^-8 relative) is inside that budget. The final fp32 state, which later decode steps
continue from, is held to 8e-3 in the fast form: about twice the largest its bf16 state
products give over these cases (4.0e-3), so that a loss of precision shows; the accurate
form to 2e-5.
"""
from __future__ import annotations

import numpy as np
import pytest

from _util import bf16_to_f32, log_case, to_dev, to_np

pytestmark = pytest.mark.gpu

PREFILL_TOL = 1e-2
STATE_TOL = 8e-3
# GDN_PREFILL_ACCURATE (V' = T' (V - e^G K S) with S, X = V - e^G K S, T' and V'' split into
# bf16 hi + lo: the state products at fp32 accuracy): measured 3e-6 to 8e-6 at every tested
# length, carried state and gate regime
STATE_TOL_ACC = 2e-5
D = 128


ACC, FAST = 0, 1  # gdn_prefill_precision: GDN_PREFILL_ACCURATE (the default), GDN_PREFILL_FAST


def run_prefill(gdn, dev, inp, Hk=16, o_dtype="bf16", precomputed=None, precision=ACC):
    import torch
    T = lambda a: None if a is None else to_dev(a, dev)  # noqa: E731
    Hv = inp.A_log.size
    kw = dict(Hk=Hk, Hv=Hv, state=T(inp.state),
              o_dtype=torch.bfloat16 if o_dtype == "bf16" else torch.float32, precision=precision)
    if inp.x is not None:
        kw.update(x=T(inp.x), conv_weight=T(inp.conv_w), conv_state=T(inp.conv_state))
    else:
        kw.update(q=T(inp.q), k=T(inp.k), v=T(inp.v))
    if precomputed is None:
        kw.update(a=T(inp.a), b=T(inp.b), A_log=T(inp.A_log), dt_bias=T(inp.dt_bias))
    else:
        kw.update(alpha=T(precomputed[0]), beta=T(precomputed[1]))
    out = gdn.prefill_chunked(**kw)
    torch.cuda.synchronize()
    o = to_np(out["o"])
    o = bf16_to_f32(o) if o_dtype == "bf16" else o
    return o, to_np(out["state"]), None if out["conv_state"] is None else to_np(out["conv_state"])


def check(O, got, ref, what, tol=PREFILL_TOL):
    r = O.rel_err(got, ref)
    m = O.max_abs(got, ref)
    print(f"  {what}: rel {r:.2e} max-abs {m:.2e}", flush=True)
    assert np.all(np.isfinite(got)), what
    assert r <= tol, (what, r)
    return r


@pytest.mark.parametrize("precision", [ACC, FAST], ids=["accurate", "fast"])
@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 130, 200])
def test_prefill_conv_against_per_token(O, gdn, dev, T, precision):
    """Conv front end, zero conv state and zero initial state (a fresh prefill), both
    precisions."""
    log_case(f"prefill conv T={T} B=1 zero state, precision {precision}")
    inp = O.make_inputs(config=4, layer=T, B=1, L=T, conv=True, conv_state=False, zero_state=True)
    ref = O.reference_layer(inp)
    o, S, conv = run_prefill(gdn, dev, inp, precision=precision)
    check(O, o, ref["o"], "o")
    check(O, S, ref["state"], "state", STATE_TOL_ACC if precision == ACC else STATE_TOL)
    assert np.array_equal(conv, ref["xp"][:, -3:])


@pytest.mark.parametrize("precision", [ACC, FAST], ids=["accurate", "fast"])
@pytest.mark.parametrize("T", [3, 100])
def test_prefill_continues_from_state_and_conv_state(O, gdn, dev, T, precision):
    """A later prefill window: non-zero state and conv state carried in, B=2."""
    log_case(f"prefill conv T={T} B=2 with state, precision {precision}")
    inp = O.make_inputs(config=4, layer=50 + T, B=2, L=T, conv=True, state_std=0.05)
    ref = O.reference_layer(inp)
    o, S, conv = run_prefill(gdn, dev, inp, o_dtype="f32", precision=precision)
    check(O, o, ref["o"], "o")
    check(O, S, ref["state"], "state", STATE_TOL)
    assert np.array_equal(conv, ref["xp"][:, -3:])


@pytest.mark.parametrize("precision", [ACC, FAST], ids=["accurate", "fast"])
def test_prefill_qkv_precomputed_gates_equal_heads(O, gdn, dev, precision):
    """qkv front end (bf16: v reordered by prefill_vfrag), alpha/beta given (delta::run's
    form), Hk = Hv = 8, a last chunk of 22 positions."""
    log_case(f"prefill qkv precomputed gates Hk=Hv=8 T=150, precision {precision}")
    inp = O.make_inputs(config=4, layer=7, B=1, L=150, Hk=8, Hv=8, state_std=0.1)
    al = O.uniform(77, (1, 150, 8), 0.85, 1.0)
    be = O.uniform(78, (1, 150, 8), 0.0, 1.0)
    q, k, v = O.from_bf16(inp.q), O.from_bf16(inp.k), O.from_bf16(inp.v)
    ro, rS = O.recurrent(q, k, v, al, be, inp.state)
    o, S, _ = run_prefill(gdn, dev, inp, Hk=8, o_dtype="f32", precomputed=(al, be), precision=precision)
    check(O, o, ro, "o")
    check(O, S, rS, "state", STATE_TOL_ACC if precision == ACC else STATE_TOL)


@pytest.mark.parametrize("Hk,Hv", [(8, 16), (4, 16), (2, 12), (4, 20)])
@pytest.mark.parametrize("precision", [ACC, FAST], ids=["accurate", "fast"])
def test_prefill_other_head_ratios(O, gdn, dev, Hk, Hv, precision):
    """Other sizes of the family: two v-heads per k-head (one group of two), four (groups of
    three and one: the intra kernel's general form), six (two full groups) and five (three
    and two); conv front end, carried state and conv state, ragged last chunk; both
    precisions."""
    log_case(f"prefill conv Hk={Hk} Hv={Hv} T=150 B=1 with state, precision {precision}")
    inp = O.make_inputs(config=4, layer=100 * Hk + Hv, B=1, L=150, Hk=Hk, Hv=Hv, conv=True,
                        state_std=0.05)
    ref = O.reference_layer(inp)
    o, S, conv = run_prefill(gdn, dev, inp, Hk=Hk, o_dtype="f32", precision=precision)
    check(O, o, ref["o"], "o")
    check(O, S, ref["state"], "state", STATE_TOL_ACC if precision == ACC else STATE_TOL)
    assert np.array_equal(conv, ref["xp"][:, -3:])


@pytest.mark.parametrize("precision", [ACC, FAST], ids=["accurate", "fast"])
def test_prefill_4096_full(O, gdn, dev, precision):
    """The benchmark configuration: B=1, T=4096, conv front end, zero state; both
    precisions."""
    log_case(f"prefill conv T=4096 B=1 (benchmark shape), precision {precision}")
    inp = O.make_inputs(config=4, layer=0, B=1, L=4096, conv=True, conv_state=False,
                        zero_state=True)
    ref = O.reference_layer(inp)
    o, S, conv = run_prefill(gdn, dev, inp, precision=precision)
    check(O, o, ref["o"], "o")
    check(O, S, ref["state"], "state", STATE_TOL_ACC if precision == ACC else STATE_TOL)
    assert np.array_equal(conv, ref["xp"][:, -3:])


def test_prefill_then_decode_continues(O, gdn, dev):
    """Prefill 130 tokens, then decode one more with the recurrent kernel: equals the
    per-token recurrence over all 131 (the segmented-prefill principle)."""
    import torch
    log_case("prefill 130 then decode 1")
    inp = O.make_inputs(config=4, layer=9, B=1, L=131, conv=True, conv_state=False,
                        zero_state=True)
    ref = O.reference_layer(inp)
    first = O.LayerInputs(None, None, None, np.ascontiguousarray(inp.x[:, :130]), inp.conv_w,
                          None, np.ascontiguousarray(inp.a[:, :130]),
                          np.ascontiguousarray(inp.b[:, :130]), inp.A_log, inp.dt_bias, None)
    _, S, conv = run_prefill(gdn, dev, first)
    state = to_dev(S, dev)
    out = gdn.layer(x=to_dev(np.ascontiguousarray(inp.x[:, 130:]), dev),
                    conv_weight=to_dev(inp.conv_w, dev), conv_state=to_dev(conv, dev),
                    a=to_dev(np.ascontiguousarray(inp.a[:, 130:]), dev),
                    b=to_dev(np.ascontiguousarray(inp.b[:, 130:]), dev),
                    A_log=to_dev(inp.A_log, dev), dt_bias=to_dev(inp.dt_bias, dev),
                    state=state, o_dtype=torch.float32)
    torch.cuda.synchronize()
    check(O, to_np(out["o"]), ref["o"][:, 130:], "decode o after prefill")
    check(O, to_np(out["state"]), ref["state"], "state after prefill + decode", STATE_TOL)


@pytest.mark.parametrize("precision", [ACC, FAST], ids=["accurate", "fast"])
def test_prefill_1024_then_decode_16(O, gdn, dev, precision):
    """A 1024-token chunked prefill (the reference's prefill window, cpp/src/session.hpp:136)
    followed by 16 single-token decode steps on the recurrent kernel, every output and the
    state after every step against the per-token recurrence over all 1040 tokens: the
    chunked form's state error is carried into decode and must not grow there. The drift
    is printed per step. Both precisions (the fp32-state form's state is held to its own,
    tighter bound)."""
    import torch
    log_case(f"prefill 1024 then decode 16, precision {precision}")
    stol = STATE_TOL_ACC if precision == ACC else STATE_TOL
    T0, N = 1024, 16
    inp = O.make_inputs(config=4, layer=11, B=1, L=T0 + N, conv=True, conv_state=False,
                        zero_state=True)
    sl = lambda a, i, j: np.ascontiguousarray(a[:, i:j])  # noqa: E731
    head = O.LayerInputs(None, None, None, sl(inp.x, 0, T0), inp.conv_w, None, sl(inp.a, 0, T0),
                         sl(inp.b, 0, T0), inp.A_log, inp.dt_bias, None)
    ref0 = O.reference_layer(head)
    o, S, conv = run_prefill(gdn, dev, head, precision=precision)
    check(O, o, ref0["o"], "prefill o")
    check(O, S, ref0["state"], "prefill state", stol)
    state, conv_d = to_dev(S, dev), to_dev(conv, dev)
    ref_state, ref_conv = ref0["state"], ref0["xp"][:, -3:]
    d = lambda a: to_dev(a, dev)  # noqa: E731
    errs = []
    for t in range(T0, T0 + N):
        step = O.LayerInputs(None, None, None, sl(inp.x, t, t + 1), inp.conv_w, ref_conv, sl(inp.a, t, t + 1),
                             sl(inp.b, t, t + 1), inp.A_log, inp.dt_bias, ref_state)
        ref = O.reference_layer(step)
        out = gdn.layer(x=d(step.x), conv_weight=d(inp.conv_w), conv_state=conv_d, a=d(step.a), b=d(step.b),
                        A_log=d(inp.A_log), dt_bias=d(inp.dt_bias), state=state, o_dtype=torch.float32)
        torch.cuda.synchronize()
        conv_d = out["conv_state"]
        eo, es = O.rel_err(to_np(out["o"]), ref["o"]), O.rel_err(to_np(state), ref["state"])
        errs.append((eo, es))
        ref_state, ref_conv = ref["state"], ref["xp"][:, -3:]
    print("  decode drift (o, state) per step: " + ", ".join(f"({a:.1e}, {b:.1e})" for a, b in errs), flush=True)
    assert max(e[0] for e in errs) <= PREFILL_TOL
    assert max(e[1] for e in errs) <= stol
    assert np.array_equal(to_np(conv_d), ref_conv)


# (T, carried state, state bound): windows of one, two and several chunks from a carried state
# (B = 2, state ~N(0, 0.05)), where a short last chunk keeps the carried state's roundings in
# K S unless S is split, and the benchmark shape
ACC_CASES = [(1, True, STATE_TOL_ACC), (65, True, STATE_TOL_ACC), (200, True, STATE_TOL_ACC),
             (4096, False, STATE_TOL_ACC)]


@pytest.mark.parametrize("T,carried,stol", ACC_CASES)
def test_prefill_accurate(O, gdn, dev, T, carried, stol):
    """GDN_PREFILL_ACCURATE against the token-by-token recurrence: the final state within the
    case's bound (S, X, T' and V'' split into bf16 hi + lo in the state products), fp32
    outputs within the chunked bound. Conv front end; with a carried state and conv state
    (B = 2, state ~N(0, 0.05)), or the benchmark shape at 4096."""
    log_case(f"prefill accurate T={T} carried={carried}")
    inp = O.make_inputs(config=4, layer=300 + T, B=2 if carried else 1, L=T, conv=True, conv_state=carried,
                        zero_state=not carried, state_std=0.05)
    ref = O.reference_layer(inp)
    o, S, conv = run_prefill(gdn, dev, inp, o_dtype="f32", precision=ACC)
    check(O, o, ref["o"], "o (fp32)")
    check(O, S, ref["state"], "state", stol)
    assert np.array_equal(conv, ref["xp"][:, -3:])


def test_prefill_accurate_slow_gates(O, gdn, dev):
    """Gates near 1 (A_log = -4: alpha in 0.93 .. 0.9997), where a chunk does not forget its
    incoming state, so every bf16 rounding in the state products persists: GDN_PREFILL_FAST
    ends about 3e-3 from the recurrence, GDN_PREFILL_ACCURATE (S split in K S, T' in T' X,
    V'' in K^T V'') within its fp32-level bound."""
    log_case("prefill T=1024 slow gates, both precisions")
    inp = O.make_inputs(config=4, layer=21, B=1, L=1024, conv=True, conv_state=False, zero_state=True)
    inp.A_log = np.full_like(inp.A_log, -4.0)
    ref = O.reference_layer(inp)
    for name, prec, tol in (("accurate", ACC, STATE_TOL_ACC), ("fast", FAST, STATE_TOL)):
        o, S, _ = run_prefill(gdn, dev, inp, o_dtype="f32", precision=prec)
        check(O, o, ref["o"], f"o (fp32, {name})")
        check(O, S, ref["state"], f"state ({name})", tol)


def _from_fragments(blocks, rows: int, cols: int):
    """A matrix stored in MFMA A-fragment order with the interleaved k order -- 16 x 32
    blocks, row block major; in a block, lane l = 16 lg + fr holds row fr, columns
    4 lg .. 4 lg + 3 (elements 0..3) and 16 + 4 lg .. 16 + 4 lg + 3 (elements 4..7) -- to
    row-major."""
    lead = blocks.shape[:-1]
    a = blocks.reshape(*lead, rows // 16, cols // 32, 4, 16, 2, 4)   # [rt][ks][lg][fr][half][e]
    n = len(lead)
    a = a.transpose(*range(n), n, n + 3, n + 1, n + 4, n + 2, n + 5)  # [rt][fr][ks][half][lg][e]
    return a.reshape(*lead, rows, cols)


def test_prefill_frontend_is_bit_exact(O, gdn, dev):
    """The prefill's own conv + SiLU + l2norm front end (fast SiLU with exact fallback)
    against the oracle's, bit for bit: Q and K^T as the intra-chunk kernel leaves them in
    the workspace (Q at offset 0, K^T after it, one 64 x 128 block per (b, k-head, chunk)
    in fragment order). B=2, a conv state carried in, T=200 (last chunk partial)."""
    import torch
    log_case("prefill front end bits B=2 T=200 with conv state")
    B, T, Hk, Hv = 2, 200, 16, 48
    inp = O.make_inputs(config=4, layer=99, B=B, L=T, conv=True, state_std=0.05)
    q_ref, k_ref, _, _ = O.conv_frontend(inp.x, inp.conv_state, inp.conv_w, Hk, Hv)
    nC = (T + 63) // 64
    ws = torch.empty(gdn.prefill_workspace_size(B, T, Hk, Hv), dtype=torch.uint8, device=dev)
    run_kw = dict(x=to_dev(inp.x, dev), conv_weight=to_dev(inp.conv_w, dev),
                  conv_state=to_dev(inp.conv_state, dev), a=to_dev(inp.a, dev), b=to_dev(inp.b, dev),
                  A_log=to_dev(inp.A_log, dev), dt_bias=to_dev(inp.dt_bias, dev),
                  state=to_dev(inp.state, dev), Hk=Hk, Hv=Hv, workspace=ws)
    gdn.prefill_chunked(**run_kw)
    torch.cuda.synchronize()
    raw = to_np(ws).view(np.uint16)
    plane = B * Hk * nC * 8192
    kt_off = -(-plane * 2 // 256) * 256 // 2
    wq = _from_fragments(raw[:plane].reshape(B, Hk, nC, 8192), 64, 128)         # [b][g][c][pos][dk]
    wkt = _from_fragments(raw[kt_off:kt_off + plane].reshape(B, Hk, nC, 8192), 128, 64)  # [b][g][c][dk][pos]
    qr = np.zeros((B, nC * 64, Hk, 128), np.uint16)
    kr = np.zeros((B, nC * 64, Hk, 128), np.uint16)
    qr[:, :T] = q_ref.view(np.uint16)
    kr[:, :T] = k_ref.view(np.uint16)
    q_got = wq.transpose(0, 2, 3, 1, 4).reshape(B, nC * 64, Hk, 128)
    k_got = wkt.transpose(0, 2, 4, 1, 3).reshape(B, nC * 64, Hk, 128)
    print(f"  q mismatches {(q_got != qr).sum()}, k mismatches {(k_got != kr).sum()}", flush=True)
    assert np.array_equal(q_got, qr)
    assert np.array_equal(k_got, kr)


def test_prefill_frontend_silu_every_finite_bf16(O, gdn, dev):
    """The front end's SiLU (hardware 2^x and reciprocal with an exact fallback) on every
    finite bf16 value, bit for bit against the oracle: conv weights (0, 0, 0, 1) make the
    conv output equal to x, the v channels of T = 16 positions hold all 65,280 finite bf16
    patterns, and v is read back from the workspace (its fragment order: block
    2 (dv / 16) + position / 32, lane 16 ((position % 16) / 4) + dv % 16, element
    position % 4 + 4 ((position % 32) / 16))."""
    import torch
    log_case("prefill front end silu on every finite bf16, B=1 T=16")
    B, T, Hk, Hv = 1, 16, 16, 48
    C = 2 * Hk * D + Hv * D
    pats = np.arange(1 << 16, dtype=np.uint32)
    finite = pats[((pats >> 7) & 0xFF) != 0xFF].astype(np.uint16)
    rng = np.random.default_rng(11)
    x = O.to_bf16(rng.standard_normal((B, T, C)).astype(np.float32))
    nv = T * Hv * D
    x[:, :, 2 * Hk * D:] = np.resize(finite, nv).reshape(1, T, Hv * D).view(x.dtype)
    w = np.zeros((4, C), np.float32)
    w[3] = 1.0
    w = O.to_bf16(w)
    _, _, v_ref, _ = O.conv_frontend(x, None, w, Hk, Hv)
    a = O.to_bf16(rng.standard_normal((B, T, Hv)).astype(np.float32))
    ws = torch.empty(gdn.prefill_workspace_size(B, T, Hk, Hv), dtype=torch.uint8, device=dev)
    gdn.prefill_chunked(x=to_dev(x, dev), conv_weight=to_dev(w, dev), a=to_dev(a, dev), b=to_dev(a, dev),
                        A_log=torch.zeros(Hv, device=dev), dt_bias=torch.zeros(Hv, device=dev),
                        Hk=Hk, Hv=Hv, workspace=ws)
    torch.cuda.synchronize()
    raw = to_np(ws).view(np.uint16)
    al = lambda n: -(-n // 256) * 256  # noqa: E731  (byte sizes of the workspace pieces)
    nC = 1
    qk, gg = B * Hk * nC * 8192 * 2, B * Hv * nC * 128 * 4
    vf_off = (2 * al(qk) + al(gg)) // 2    # after Q, K^T and the gate factors
    vf = raw[vf_off:vf_off + Hv * 8192].reshape(Hv, 8192)
    pos = np.arange(T)[:, None]
    dv = np.arange(D)[None, :]
    idx = ((2 * (dv >> 4) + (pos >> 5)) * 512 + (16 * ((pos & 15) >> 2) + (dv & 15)) * 8
           + (pos & 3) + 4 * ((pos & 31) >> 4))
    v_got = vf[:, idx].transpose(1, 0, 2)                      # (T, Hv, D)
    v_want = v_ref.view(np.uint16)[0]
    bad = int((v_got != v_want).sum())
    print(f"  {finite.size} finite inputs, mismatches {bad}", flush=True)
    assert bad == 0


def test_prefill_timed_equals_untimed(O, gdn, dev):
    """gdn_prefill_chunked_timed runs the same kernels as gdn_prefill_chunked (identical
    outputs) and reports three positive kernel durations."""
    import torch
    log_case("prefill timed vs untimed, T=300 conv")
    T = 300
    inp = O.make_inputs(config=4, layer=7, B=1, L=T, conv=True, conv_state=False, zero_state=True)
    d = lambda a: to_dev(a, dev)  # noqa: E731
    outs = []
    for timed in (False, True):
        o = torch.empty((1, T, 48, D), dtype=torch.bfloat16, device=dev)
        st = torch.empty((1, 48, D, D), device=dev)
        ws = torch.empty(gdn.prefill_workspace_size(1, T), dtype=torch.uint8, device=dev)
        args = gdn.layer_args(B=1, T=T, x=d(inp.x), conv_weight=d(inp.conv_w), a=d(inp.a), b=d(inp.b),
                              A_log=d(inp.A_log), dt_bias=d(inp.dt_bias), state_out=st, o=o, workspace=ws)
        if timed:
            ms = gdn.call_prefill_timed(args)
            print(f"  kernel ms {ms}", flush=True)
            assert len(ms) == 3 and all(m > 0 for m in ms), ms
        else:
            gdn.call_prefill(args)
        torch.cuda.synchronize()
        outs.append((o.clone(), st.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
