"""Benchmark of the gated-delta recurrence on one MI355X.

The headline (`value`) is the 48-layer, B=1 decode step with the conv front end: one
gdn_run call over 48 independent layers, each with its own fp32 state (151 MB of state
read and written per step). Reported as algorithmic GB/s:
    313,420,800 B per step = 48 x (6,291,456 state r+w + 238,144 front end, gates, o).
Secondary lines: B=32 decode (9,714,321,408 B per step), speculative verify (B=8, T=5,
152,887,168 B), and chunked prefill T=4096 (tokens/s, intra-chunk MFMA FLOP rate).

State sets are rotated so the working set exceeds the 256 MB last-level cache: every
timed step streams its state from HBM. The CPU baseline runs the oracle's unfused,
one-pass-per-op restatement of the same step on the host cores.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E, AMD spec
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16
D = 128
HK, HV = 16, 48
C = 2 * HK * D + HV * D          # 10240 conv channels
METRIC = "gated-delta decode state GB/s (% HBM peak) at B=1,32; prefill tok/s T=4096"
# Plain memory streams with the kernels' traffic shapes (the ceilings the decode and verify
# rates are read against): bench instrumentation, not part of the library.
PROBE_SRC = os.path.join(ROOT, "stream_probe.hip")
PROBE_LIB = os.path.join(ROOT, "libstream_probe.so")


def build_probe(verbose: bool = False) -> str:
    """Compile stream_probe.hip into libstream_probe.so beside this file (with the library's
    HIP flags); __graft_entry__.build() calls it."""
    import importlib.util
    import subprocess
    spec = importlib.util.spec_from_file_location("gdn_bench_build_flags",
                                                  os.path.join(ROOT, "qwen3.8-27b-mlx_amd", "_build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    tmp = PROBE_LIB + ".tmp"
    cmd = [mod.hipcc(), *mod.HIPCC_FLAGS, "-shared", "-o", tmp, PROBE_SRC]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"probe build failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def bytes_decode_layer(B: int, conv: bool) -> int:
    """Algorithmic bytes of one layer's decode step (state r+w, inputs, outputs)."""
    state = B * HV * D * D * 4 * 2
    gates = B * HV * 2 * 2 + HV * 4 * 2          # a, b bf16; A_log, dt_bias fp32
    o = B * HV * D * 2                            # bf16
    if conv:
        front = B * C * 2 + B * 3 * C * 2 * 2 + 4 * C * 2   # x, conv state r+w, conv w
    else:
        front = B * 2 * HK * D * 2 + B * HV * D * 2         # q, k, v bf16
    return state + gates + o + front


def bytes_verify(B: int, T: int) -> int:
    state_read = B * HV * D * D * 4
    states = B * HV * T * D * D * 4
    x = B * T * C * 2
    conv_state = B * 3 * C * 2
    w = 4 * C * 2
    ab = B * T * HV * 2 * 2
    params = HV * 4 * 2
    o = B * T * HV * D * 2
    return state_read + states + x + conv_state + w + ab + params + o


def make_layer_inputs(torch, dev, nl: int, B: int, T: int, conv: bool, seed: int):
    """Synthetic inputs with the benchmark distributions (torch RNG on the device)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    n = lambda *s: torch.randn(s, device=dev, generator=g)  # noqa: E731

    def unit_bf16(*s):
        x = n(*s)
        return (x / x.norm(dim=-1, keepdim=True)).to(torch.bfloat16)

    q = unit_bf16(nl, B, T, HK, D)
    k = unit_bf16(nl, B, T, HK, D)
    v = n(nl, B, T, HV, D).to(torch.bfloat16)
    inp = dict(
        a=n(nl, B, T, HV).to(torch.bfloat16),
        b=n(nl, B, T, HV).to(torch.bfloat16),
        A_log=torch.rand((nl, HV), device=dev, generator=g) * 2 - 1,
        dt_bias=n(nl, HV) * 0.1,
    )
    if conv:
        inp["x"] = torch.cat([q.reshape(nl, B, T, HK * D), k.reshape(nl, B, T, HK * D),
                              v.reshape(nl, B, T, HV * D)], dim=-1).contiguous()
        inp["conv_weight"] = (n(nl, 4, C) * 0.1).to(torch.bfloat16)
        inp["conv_state"] = n(nl, B, 3, C).to(torch.bfloat16)
    else:
        inp.update(q=q, k=k, v=v)
    return inp


class Timer:
    """HIP events on torch's current stream (the stream the library launches on).

    Before the timed launches are enqueued, the stream is held by a spin kernel long
    enough for the host to enqueue all of them, so the event pairs bracket GPU work only
    (host-side launch overhead would otherwise leave the GPU idle between short kernels).
    """

    def __init__(self, torch):
        self.torch = torch
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        torch.cuda.synchronize()
        s.record()
        torch.cuda._sleep(2_000_000)
        e.record()
        torch.cuda.synchronize()
        self.cycles_per_ms = 2_000_000 / max(s.elapsed_time(e), 1e-3)

    def hold(self, ms: float):
        self.torch.cuda._sleep(int(self.cycles_per_ms * ms))

    def time_calls(self, fn, steps: int, warmup: int, host_us_per_call: float = 60.0):
        """Two passes of `steps` calls after `warmup`: the whole job (the calls back to
        back, one event pair around all of them: ms_per_step) and then each call between
        its own event pair (launch_ms_*, reported beside it: those timing packets add
        about 2 us per call, so they are kept out of the whole-job pass)."""
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        self.hold(2.0 + steps * host_us_per_call * 1e-3)
        t0.record()
        for i in range(steps):
            fn(warmup + i)
        t1.record()
        torch.cuda.synchronize()
        total = t0.elapsed_time(t1)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        self.hold(2.0 + steps * host_us_per_call * 1e-3)
        for i in range(steps):
            evs[i][0].record()
            fn(warmup + steps + i)
            evs[i][1].record()
        torch.cuda.synchronize()
        per = sorted(a.elapsed_time(b) for a, b in evs)
        return dict(ms_per_step=total / steps, launch_ms_avg=sum(per) / len(per),
                    launch_ms_p10=per[len(per) // 10], launch_ms_p50=per[len(per) // 2],
                    launch_ms_p90=per[(9 * len(per)) // 10])


def bench_decode(torch, gdn, dev, timer, B: int, conv: bool, steps: int, warmup: int,
                 sets: int, NL: int = 48):
    """NL-layer decode step, rotating over `sets` independent state sets."""
    inps = [make_layer_inputs(torch, dev, NL, B, 1, conv, seed=100 + s) for s in range(sets)]
    states = []
    for s in range(sets):
        g = torch.Generator(device=dev)
        g.manual_seed(900 + s)
        states.append(torch.randn((NL, B, HV, D, D), device=dev, generator=g) * 0.02)
    o = torch.empty((NL, B, 1, HV, D), dtype=torch.bfloat16, device=dev)
    conv_out = ([torch.empty((NL, B, 3, C), dtype=torch.bfloat16, device=dev) for _ in range(sets)]
                if conv else [None] * sets)
    argsets = []
    for s in range(sets):
        i = inps[s]
        argsets.append(gdn.layer_args(
            B=B, T=1, n_layers=NL, q=i.get("q"), k=i.get("k"), v=i.get("v"), x=i.get("x"),
            conv_weight=i.get("conv_weight"), conv_state_in=i.get("conv_state"),
            conv_state_out=conv_out[s], a=i["a"], b=i["b"], A_log=i["A_log"],
            dt_bias=i["dt_bias"], state_in=states[s], state_out=states[s], o=o))
    fn = lambda it: gdn.call_run(argsets[it % sets])  # noqa: E731
    r = timer.time_calls(fn, steps, warmup)
    nbytes = NL * bytes_decode_layer(B, conv)
    r["bytes_per_step"] = nbytes
    r["GBps"] = nbytes / (r["ms_per_step"] * 1e-3) / 1e9
    r["kernel_GBps"] = nbytes / (r["launch_ms_avg"] * 1e-3) / 1e9
    r["state_sets"] = sets
    r["working_set_MB"] = sets * NL * B * HV * D * D * 4 / 1e6
    del states, inps
    return r


def bench_verify(torch, gdn, dev, timer, steps: int, warmup: int, sets: int):
    B, T = 8, 5
    inps = [make_layer_inputs(torch, dev, 1, B, T, True, seed=300 + s) for s in range(sets)]
    states_in = [torch.randn((1, B, HV, D, D), device=dev) * 0.02 for _ in range(sets)]
    outs = [torch.empty((1, B, HV, T, D, D), device=dev) for _ in range(sets)]
    o = torch.empty((1, B, T, HV, D), dtype=torch.bfloat16, device=dev)
    argsets = []
    for s in range(sets):
        i = inps[s]
        argsets.append(gdn.layer_args(
            B=B, T=T, x=i["x"], conv_weight=i["conv_weight"], conv_state_in=i["conv_state"],
            a=i["a"], b=i["b"], A_log=i["A_log"], dt_bias=i["dt_bias"], state_in=states_in[s],
            states=outs[s], o=o))
    r = timer.time_calls(lambda it: gdn.call_run(argsets[it % sets]), steps, warmup)
    nbytes = bytes_verify(B, T)
    r["bytes_per_step"] = nbytes
    r["GBps"] = nbytes / (r["ms_per_step"] * 1e-3) / 1e9
    r["kernel_GBps"] = nbytes / (r["launch_ms_avg"] * 1e-3) / 1e9
    return r


# Chunked prefill, T=4096, chunk 64: normative FLOP counts of the intra-chunk products
# (Gram K K^T and scores Q K^T per k-head; W = T(beta g K), U = T(beta V) and the intra
# output (Q K^T . Gamma) V' per v-head) and of the inter-chunk state products.
def prefill_flops(T: int, C: int = 64):
    nC = T // C
    intra = nC * (HK * 2 * 2 * C * C * D + HV * 3 * 2 * C * C * D)
    inter = nC * HV * 3 * 2 * C * D * D
    return intra, inter


def bench_prefill(torch, gdn, dev, timer, steps: int, warmup: int, T: int = 4096, precision: int = 0):
    """One layer, B = 1, conv front end; `precision` is gdn_prefill_precision (0, the default,
    carries the state products at fp32 accuracy through bf16 hi + lo splits; 1 is the fast
    form, bf16 operands)."""
    i = make_layer_inputs(torch, dev, 1, 1, T, True, seed=500)
    x = i["x"][0].contiguous()
    o = torch.empty((1, T, HV, D), dtype=torch.bfloat16, device=dev)
    state_out = torch.empty((1, HV, D, D), device=dev)
    conv_out = torch.empty((1, 3, C), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(gdn.prefill_workspace_size(1, T, precision=precision), dtype=torch.uint8, device=dev)
    args = gdn.layer_args(B=1, T=T, x=x, conv_weight=i["conv_weight"][0].contiguous(),
                          conv_state_in=None, conv_state_out=conv_out, a=i["a"][0].contiguous(),
                          b=i["b"][0].contiguous(), A_log=i["A_log"][0].contiguous(),
                          dt_bias=i["dt_bias"][0].contiguous(), state_in=None,
                          state_out=state_out, o=o, workspace=ws, precision=precision)
    r = timer.time_calls(lambda it: gdn.call_prefill(args), steps, warmup, host_us_per_call=80.0)
    intra, inter = prefill_flops(T)
    sec = r["ms_per_step"] * 1e-3
    traffic = load_traffic("prefill_t4096_b1_conv") if T == 4096 and precision == 0 else None
    # each kernel between its own event pair (gdn_prefill_chunked_timed; outside the timed
    # region above: every such call waits for its events). A short spin queued ahead of each
    # call keeps the stream busy while the call is enqueued, so that the first kernel's
    # pair does not also time the launch from an idle queue.
    per = []
    for _ in range(max(steps, 10)):
        timer.hold(0.3)
        per.append(gdn.call_prefill_timed(args))
    event_us = [sorted(p[i] for p in per)[len(per) // 2] * 1e3 for i in range(3)]
    return dict(tokens_per_s=T / sec, us_per_call=r["ms_per_step"] * 1e3,
                intra_TFLOPs=intra / sec / 1e12,
                intra_frac_mfma=intra / sec / (MFMA_BF16_PEAK_TFLOPS * 1e12),
                all_products_frac_mfma=(intra + inter) / sec / (MFMA_BF16_PEAK_TFLOPS * 1e12),
                intra_flop=intra, inter_flop=inter,
                hbm_bytes=traffic, hbm_GBps=None if traffic is None else traffic / sec / 1e9,
                per_kernel=prefill_kernel_fracs(event_us) if T == 4096 and precision == 0 else None,
                event_us=[round(u, 2) for u in event_us])


def prefill_kernel_fracs(event_us=None):
    """MFMA fraction of each prefill kernel alone: its normative and executed MFMA FLOPs
    (from the committed counter run) over its own duration, against the dense bf16 peak --
    the duration measured in this run between the kernel's own event pair (event_us: front
    end, intra, scan, from gdn_prefill_chunked_timed) and, beside it, the committed
    rocprofv3 kernel-trace average with the busy-cycle counter."""
    path = os.path.join(ROOT, "profiles", "prefill_kernels.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        ks = json.load(fh)["kernels"]
    peak = MFMA_BF16_PEAK_TFLOPS * 1e12
    order = ("prefill_frontend_kernel", "prefill_intra_kernel", "prefill_scan_kernel")
    out = {}
    for i, name in enumerate(order):
        k = ks[name]
        s = k["avg_us"] * 1e-6
        d = dict(avg_us=k["avg_us"], frac_mfma_normative=round(k["normative_flop"] / s / peak, 4),
                 frac_mfma_executed=round(k["executed_mfma_flop"] / s / peak, 4),
                 mfma_busy_counter=k["mfma_busy"])
        if event_us is not None:
            se = event_us[i] * 1e-6
            d.update(event_us=round(event_us[i], 2),
                     frac_mfma_normative_event=round(k["normative_flop"] / se / peak, 4),
                     frac_mfma_executed_event=round(k["executed_mfma_flop"] / se / peak, 4))
        out[name] = d
    return out


def bench_crossover(torch, gdn, dev, timer, steps: int, warmup: int, Ts=(16, 32, 64, 128, 256, 512, 1024),
                    Bs=(1, 4)):
    """One layer with the conv front end over T tokens, B sequences: the recurrent kernel
    (gdn_run, serial in T) against the chunked prefill (gdn_prefill_chunked), us per call.
    The crossover is where a non-recording call switches forms (the reference makes the same
    choice by length, python/qwen35.py:606-626)."""
    out = {}
    for B in Bs:
        for T in Ts:
            i = make_layer_inputs(torch, dev, 1, B, T, True, seed=800 + T + B)
            x = i["x"][0].contiguous()
            cw = i["conv_weight"][0].contiguous()
            a, b = i["a"][0].contiguous(), i["b"][0].contiguous()
            A_log, dt_bias = i["A_log"][0].contiguous(), i["dt_bias"][0].contiguous()
            state = torch.randn((B, HV, D, D), device=dev) * 0.02
            o = torch.empty((B, T, HV, D), dtype=torch.bfloat16, device=dev)
            conv_out = torch.empty((B, 3, C), dtype=torch.bfloat16, device=dev)
            st_out = torch.empty_like(state)
            ws = torch.empty(gdn.prefill_workspace_size(B, T), dtype=torch.uint8, device=dev)
            common = dict(B=B, T=T, x=x, conv_weight=cw, conv_state_in=i["conv_state"][0].contiguous(),
                          conv_state_out=conv_out, a=a, b=b, A_log=A_log, dt_bias=dt_bias, state_in=state,
                          state_out=st_out, o=o)
            rec = gdn.layer_args(**common)
            chk = gdn.layer_args(**common, workspace=ws)
            n = max(5, steps // 4)
            r1 = timer.time_calls(lambda it: gdn.call_run(rec), n, warmup, host_us_per_call=80.0)
            r2 = timer.time_calls(lambda it: gdn.call_prefill(chk), n, warmup, host_us_per_call=80.0)
            out[f"B{B}_T{T}"] = dict(recurrent_us=round(r1["ms_per_step"] * 1e3, 1),
                                     chunked_us=round(r2["ms_per_step"] * 1e3, 1))
            print(f"# crossover B={B} T={T}: recurrent {r1['ms_per_step'] * 1e3:.1f} us, "
                  f"chunked {r2['ms_per_step'] * 1e3:.1f} us", flush=True)
    return out


def bench_qlinear(torch, gdn, dev, timer, steps: int, warmup: int, which: str, M: int = 1, NL: int = 48):
    """NL layers (48: a model's DeltaNet layers) of the projections for M operand rows in one
    launch (M = 1: B=1 decode, the GEMV kernel; M = 40: a B=8, T=5 verify block, and M = 1024
    with NL = 1: one layer's prefill window, the MFMA kernel): "in_proj" = in_proj_qkv,
    in_proj_z, in_proj_a, in_proj_b on x (5120); "out_proj" = GatedRMSNorm of o (6144, fp32)
    with z, then out_proj (5120 rows). Synthetic 4-bit weights (random words, scales and
    biases in the checkpoint's ranges)."""
    g = torch.Generator(device=dev)
    g.manual_seed(700 if which == "in_proj" else 701)

    def mat(n, k):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (NL, n, k // 8), dtype=torch.int32, device=dev, generator=g)
        sc = (torch.rand((NL, n, k // 64), device=dev, generator=g) * 0.03 + 0.002).to(torch.bfloat16)
        bi = ((torch.rand((NL, n, k // 64), device=dev, generator=g) - 0.5) * 0.4).to(torch.bfloat16)
        return gdn.QuantLinear(w, sc, bi)

    if which == "in_proj":
        K, ns = 5120, [C, HV * D, HV, HV]
        mats = [mat(n, K) for n in ns]
        x = torch.randn((NL, M, K), device=dev, generator=g).to(torch.bfloat16)
        args, _ys = gdn.qlinear_args(mats, x, n_layers=NL)
        operand = K * 2
    else:
        K, ns = HV * D, [5120]
        mats = [mat(n, K) for n in ns]
        o = torch.randn((NL, M, K), device=dev, generator=g) * 0.3
        z = torch.randn((NL, M, K), device=dev, generator=g).to(torch.bfloat16)
        gamma = torch.rand((NL, D), device=dev, generator=g) + 0.5
        args, _ys = gdn.qlinear_args(mats, norm=(o, z, gamma, 1e-6), n_layers=NL)
        operand = K * 4 + K * 2 + D * 4
    r = timer.time_calls(lambda it: gdn.call_qlinear(args), steps, warmup)
    # algorithmic bytes: weights, scales and biases once, the operand and the outputs (the
    # MFMA path's workspace round trip is not counted)
    per_layer = sum(n * K // 2 + n * (K // 64) * 4 + M * n * 2 for n in ns) + M * operand
    nbytes = NL * per_layer
    flop = NL * 2 * M * K * sum(ns)
    out = dict(M=M, GBps=round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9, 1),
               frac_hbm=round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
               us_per_step=round(r["ms_per_step"] * 1e3, 2), bytes_per_step=nbytes,
               TFLOPs=round(flop / (r["ms_per_step"] * 1e-3) / 1e12, 2))
    if M == 1:
        out["traffic"] = load_traffic("in_proj_48_layers_b1" if which == "in_proj" else "out_proj_norm_48_layers_b1")
    return out


def bench_copy_ceiling(torch, dev, timer, steps: int = 50):
    """Device-to-device copy of 604 MB: a practical streaming ceiling for comparison."""
    n = 4 * 48 * HV * D * D // 2
    src = [torch.empty(n, device=dev) for _ in range(2)]
    dst = [torch.empty(n, device=dev) for _ in range(2)]
    r = timer.time_calls(lambda it: dst[it % 2].copy_(src[it % 2]), steps, 5)
    return dict(GBps=2 * n * 4 / (r["ms_per_step"] * 1e-3) / 1e9, bytes=2 * n * 4)


def stream_ceilings(torch, dev, timer, steps: int, b32: bool = False):
    """Plain memory streams with the decode and verify state traffic's shapes (libstream_probe.so,
    no arithmetic): the decode step's 4,608 tiles of 32 KB read and written back in place
    (302 MB); the same with each workgroup also moving its share of the front end's bytes
    (x, conv state read and written, conv weights, gate inputs, o: the step's full
    313.4 MB); the 302 MB read only and written only; and verify's 768 tiles read once and
    written 5 times -- each rotated over 8 buffer sets as the kernels' lines are. With b32,
    the B=32 step's 147,456 tiles over 2 sets. The kernels' rates are read against these."""
    import ctypes
    if not os.path.exists(PROBE_LIB):
        return None
    L = ctypes.CDLL(PROBE_LIB)
    L.gdn_probe_rmw.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    L.gdn_probe_rmw_split.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    L.gdn_probe_rmw_groups.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.gdn_probe_read_write_t.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p]
    L.gdn_probe_rmw_fe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.gdn_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    L.gdn_probe_write.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    tile = 8192  # floats (32 KB)
    out = {}
    nd = 48 * HV * 2  # decode: 48 layers x 48 heads x two 64-row tiles
    bufs = [torch.randn(nd * tile, device=dev) for _ in range(8)]
    r = timer.time_calls(lambda it: L.gdn_probe_rmw(bufs[it % 8].data_ptr(), nd, st()), steps, 10)
    nbytes = 2 * nd * tile * 4
    out["decode_shape_rmw_stream"] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                                          GBps=round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9, 1), bytes=nbytes)
    # in the kernel's order: the 6 tiles of a k-head (3 v-heads x 2) per XCD turn
    r = timer.time_calls(lambda it: L.gdn_probe_rmw_groups(bufs[it % 8].data_ptr(), nd, 6, st()), steps, 10)
    out["decode_shape_rmw_stream_kheads"] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                                                 GBps=round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9, 1), bytes=nbytes)
    # the step's full bytes: per layer the front end reads 164,416 B (x, conv state, conv
    # weights, a, b, A_log, dt_bias) and writes 73,728 B (conv state, o), which over the
    # layer's 96 tiles is 107 float4 read and 48 written per tile (313,417,728 B per step
    # against the kernel's 313,420,800)
    fe_rd, fe_wr = 107, 48
    fe_in = [torch.randn(nd * fe_rd * 4, device=dev) for _ in range(8)]
    fe_out = [torch.empty(nd * fe_wr * 4, device=dev) for _ in range(8)]
    r = timer.time_calls(lambda it: L.gdn_probe_rmw_fe(bufs[it % 8].data_ptr(), fe_in[it % 8].data_ptr(),
                                                       fe_out[it % 8].data_ptr(), nd, fe_rd, fe_wr, 6, st()), steps, 10)
    fb = nbytes + nd * (fe_rd + fe_wr) * 16
    out["decode_full_bytes_rmw_stream"] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                                               GBps=round(fb / (r["ms_per_step"] * 1e-3) / 1e9, 1), bytes=fb)
    del fe_in, fe_out
    sink = torch.zeros(1, device=dev)
    r = timer.time_calls(lambda it: L.gdn_probe_read(bufs[it % 8].data_ptr(), sink.data_ptr(), nd, st()), steps, 10)
    out["decode_shape_read_stream"] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                                           GBps=round(nbytes / 2 / (r["ms_per_step"] * 1e-3) / 1e9, 1),
                                           bytes=nbytes // 2)
    r = timer.time_calls(lambda it: L.gdn_probe_write(bufs[it % 8].data_ptr(), nd, st()), steps, 10)
    out["decode_shape_write_stream"] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                                            GBps=round(nbytes / 2 / (r["ms_per_step"] * 1e-3) / 1e9, 1),
                                            bytes=nbytes // 2)
    del bufs
    if b32:
        # the B=32 step's state traffic: 147,456 tiles (4.8 GB) over 2 sets, as its bench line,
        # in dispatch order and split into a contiguous eighth per XCD (the kernel's order)
        nb = 32 * nd
        bufs = [torch.empty(nb * tile, device=dev).uniform_() for _ in range(2)]
        nbytes = 2 * nb * tile * 4
        for key, fn in (("decode_b32_shape_rmw_stream", L.gdn_probe_rmw),
                        ("decode_b32_shape_rmw_stream_split", L.gdn_probe_rmw_split)):
            r = timer.time_calls(lambda it: fn(bufs[it % 2].data_ptr(), nb, st()), max(10, steps // 2), 3)
            out[key] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                            GBps=round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9, 1), bytes=nbytes)
        del bufs
    nv, T = 8 * HV * 2, 5  # verify: B=8 x 48 heads x two tiles, 5 per-step states
    src = [torch.randn(nv * tile, device=dev) for _ in range(8)]
    dst = [torch.empty(nv * T * tile, device=dev) for _ in range(8)]
    r = timer.time_calls(lambda it: L.gdn_probe_read_write_t(src[it % 8].data_ptr(), dst[it % 8].data_ptr(), nv, T, st()),
                         steps, 10)
    nbytes = (1 + T) * nv * tile * 4
    out["verify_shape_stream"] = dict(us=round(r["ms_per_step"] * 1e3, 2),
                                      GBps=round(nbytes / (r["ms_per_step"] * 1e-3) / 1e9, 1), bytes=nbytes)
    return out


def launch_floors(torch, dev, timer, steps: int):
    """What a one-layer launch cannot beat, timed the same way: a one-element kernel (the
    launch itself), a device copy of one layer's 3.1 MB state (3.1 MB read + 3.1 MB
    written), and the same state read and written back in place by the decode kernel's
    one-layer grid (384 workgroups of 16-row tiles in its XCD order, libstream_probe.so),
    each back to back over rotating buffers."""
    one = torch.zeros(1, device=dev)
    r = timer.time_calls(lambda it: one.add_(1), steps, 20)
    n = HV * D * D
    src = [torch.randn(n, device=dev) for _ in range(48)]
    dst = [torch.empty(n, device=dev) for _ in range(48)]
    c = timer.time_calls(lambda it: dst[it % 48].copy_(src[it % 48]), steps, 20)
    out = dict(empty_kernel_us=round(r["ms_per_step"] * 1e3, 2),
               copy_one_layer_state_us=round(c["ms_per_step"] * 1e3, 2))
    del src, dst
    if os.path.exists(PROBE_LIB):
        import ctypes
        L = ctypes.CDLL(PROBE_LIB)
        L.gdn_probe_rmw_small.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        tiles, group = HV * (D // 16), (HV // HK) * (D // 16)  # 384 tiles of 8 KB, 24 per k-head
        bufs = [torch.randn(n, device=dev) for _ in range(96)]
        st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
        if L.gdn_probe_rmw_small(bufs[0].data_ptr(), tiles, group, st()) != 0:
            raise RuntimeError("gdn_probe_rmw_small failed")
        m = timer.time_calls(lambda it: L.gdn_probe_rmw_small(bufs[it % 96].data_ptr(), tiles, group, st()),
                             steps, 20)
        out["rmw_one_layer_state_us"] = round(m["ms_per_step"] * 1e3, 2)
    return out


def cpu_baseline(target_seconds: float = 12.0):
    """The oracle's unfused op sequence for the 48-layer B=1 decode step with the conv
    front end (one full pass per op over materialised temporaries), on the host cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = len(os.sched_getaffinity(0))
    inps = [O.make_inputs(config=1, layer=l, B=1, L=1, conv=True) for l in range(48)]
    O.reference_layer(inps[0], materialize=True, threads=threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        for inp in inps:
            O.reference_layer(inp, materialize=True, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_seconds or reps >= 200:
            break
    per_step = el / reps
    # and on one core, a shorter sample
    reps1, t0 = 0, time.perf_counter()
    while True:
        for inp in inps:
            O.reference_layer(inp, materialize=True, threads=1)
        reps1 += 1
        el1 = time.perf_counter() - t0
        if el1 >= target_seconds / 3 or reps1 >= 50:
            break
    per_step1 = el1 / reps1
    nbytes = 48 * bytes_decode_layer(1, True)
    return dict(value=nbytes / per_step / 1e9, unit="GB/s", cores=threads, kind="port",
                sample=f"{reps} full 48-layer B=1 decode steps with the conv front end "
                       f"(oracle, one pass per op, fp32), {per_step * 1e3:.1f} ms per step",
                value_1core=nbytes / per_step1 / 1e9,
                sample_1core=f"{reps1} steps on one thread, {per_step1 * 1e3:.1f} ms per step")


def load_traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 counter runs (profiles/)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        entry = json.load(fh).get(name)
    return None if entry is None else entry["bytes"]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="",
                    help="comma list: decode1,decode1layer,decode32,verify,prefill,in_proj,"
                         "out_proj,in_proj40,out_proj40,in_proj1024,out_proj1024,copy; crossover runs "
                         "only when named")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the gated-delta path "
                                   "needs no collectives; use --gpus 1"}))
        return 2

    import torch
    import __graft_entry__
    gdn = __graft_entry__.load_package()
    if not torch.cuda.is_available() or not gdn.available():
        print(json.dumps({"error": "no gfx950 GPU visible"}))
        return 1
    dev = torch.device("cuda:0")
    timer = Timer(torch)
    only = set(filter(None, args.only.split(",")))
    want = lambda n: not only or n in only  # noqa: E731

    sec = {}
    head = None
    if want("decode1"):
        # 8 state sets (1.2 GB, against the 256 MB last-level cache) for the headline; the
        # same step over 4 sets (604 MB) beside it
        head = bench_decode(torch, gdn, dev, timer, B=1, conv=True, steps=args.steps,
                            warmup=args.warmup, sets=8)
        print(f"# decode B=1 x48 conv, 8 state sets: {head['ms_per_step'] * 1e3:.1f} us/step, "
              f"{head['GBps']:.0f} GB/s", flush=True)
        r4 = bench_decode(torch, gdn, dev, timer, B=1, conv=True, steps=args.steps,
                          warmup=args.warmup, sets=4)
        sec["decode_b1_48_layers_4_sets"] = dict(
            GBps=round(r4["GBps"], 1), frac_hbm=round(r4["GBps"] / HBM_PEAK_GBPS, 4),
            us_per_step=round(r4["ms_per_step"] * 1e3, 2), working_set_MB=round(r4["working_set_MB"], 1))
        print(f"# decode B=1 x48 conv, 4 state sets: {r4['ms_per_step'] * 1e3:.1f} us/step, "
              f"{r4['GBps']:.0f} GB/s", flush=True)
    if want("decode1layer"):
        # one layer per launch (the reference's per-layer call): q, k, v given, and with the
        # conv front end at B = 1, 2; 96 / B state sets (302 MB)
        for name, B, conv in (("decode_1layer_b1", 1, False), ("decode_1layer_b1_conv", 1, True),
                              ("decode_1layer_b2_conv", 2, True)):
            r = bench_decode(torch, gdn, dev, timer, B=B, conv=conv, steps=args.steps,
                             warmup=args.warmup, sets=96 // B, NL=1)
            sec[name] = dict(GBps=round(r["GBps"], 1), frac_hbm=round(r["GBps"] / HBM_PEAK_GBPS, 4),
                             us_per_step=round(r["ms_per_step"] * 1e3, 2), bytes_per_step=r["bytes_per_step"])
            print(f"# decode 1 layer B={B}{' conv' if conv else ''}: {r['ms_per_step'] * 1e3:.2f} us/step, "
                  f"{r['GBps']:.0f} GB/s", flush=True)
        sec["launch_floors"] = launch_floors(torch, dev, timer, args.steps)
    if want("decode32"):
        r = bench_decode(torch, gdn, dev, timer, B=32, conv=False,
                         steps=max(10, args.steps // 10), warmup=3, sets=2)
        sec["decode_b32_48_layers"] = dict(
            GBps=round(r["GBps"], 1), frac_hbm=round(r["GBps"] / HBM_PEAK_GBPS, 4),
            ms_per_step=round(r["ms_per_step"], 4), bytes_per_step=r["bytes_per_step"])
        print(f"# decode B=32 x48: {r['ms_per_step']:.3f} ms/step, {r['GBps']:.0f} GB/s", flush=True)
    if want("verify"):
        # 8 sets: 1.2 GB of per-step states and states, beyond the last-level cache
        r = bench_verify(torch, gdn, dev, timer, steps=args.steps, warmup=args.warmup, sets=8)
        sec["verify_b8_t5"] = dict(GBps=round(r["GBps"], 1), frac_hbm=round(r["GBps"] / HBM_PEAK_GBPS, 4),
                                   us_per_call=round(r["ms_per_step"] * 1e3, 2),
                                   bytes_per_call=r["bytes_per_step"], traffic=load_traffic("verify_b8_t5"))
        print(f"# verify B=8 T=5: {r['ms_per_step'] * 1e3:.1f} us, {r['GBps']:.0f} GB/s", flush=True)
    if want("prefill"):
        r = bench_prefill(torch, gdn, dev, timer, steps=max(5, args.steps // 10), warmup=3)
        sec["prefill_t4096"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        hbm = "" if r["hbm_GBps"] is None else f", HBM {r['hbm_GBps']:.0f} GB/s (counted bytes)"
        print(f"# prefill T=4096: {r['us_per_call']:.1f} us, {r['tokens_per_s'] / 1e6:.2f} M tok/s, "
              f"intra MFMA frac {r['intra_frac_mfma']:.4f}{hbm}", flush=True)
        pk = r["per_kernel"]
        if pk and "event_us" in pk["prefill_intra_kernel"]:
            ki, ks = pk["prefill_intra_kernel"], pk["prefill_scan_kernel"]
            print(f"# prefill kernels (events): front end {pk['prefill_frontend_kernel']['event_us']:.1f} us, "
                  f"intra {ki['event_us']:.1f} us (MFMA {ki['frac_mfma_normative_event']:.4f} normative, "
                  f"{ki['frac_mfma_executed_event']:.4f} executed), scan {ks['event_us']:.1f} us "
                  f"({ks['frac_mfma_executed_event']:.4f} executed)", flush=True)
        # the fast form (GDN_PREFILL_FAST: bf16 S, T' and V'' in the state products) beside it
        rf = bench_prefill(torch, gdn, dev, timer, steps=max(5, args.steps // 10), warmup=3, precision=1)
        sec["prefill_t4096_fast"] = dict(us_per_call=round(rf["us_per_call"], 2),
                                         tokens_per_s=round(rf["tokens_per_s"], 1),
                                         intra_frac_mfma=round(rf["intra_frac_mfma"], 4),
                                         event_us=rf["event_us"])
        print(f"# prefill T=4096 fast form: {rf['us_per_call']:.1f} us (kernels {rf['event_us']} us)", flush=True)
    for which in ("in_proj", "out_proj"):
        if want(which):
            r = bench_qlinear(torch, gdn, dev, timer, steps=max(10, args.steps // 4), warmup=5, which=which)
            sec[f"{which}_48_layers_b1"] = r
            print(f"# {which} x48 B=1 (4-bit): {r['us_per_step']:.1f} us/step, {r['GBps']:.0f} GB/s", flush=True)
        if want(which + "1024"):
            r = bench_qlinear(torch, gdn, dev, timer, steps=max(10, args.steps // 8), warmup=3, which=which, M=1024,
                              NL=1)
            sec[f"{which}_1_layer_m1024"] = r
            print(f"# {which} x1 M=1024 (4-bit, MFMA): {r['us_per_step']:.1f} us/step, {r['TFLOPs']:.1f} TFLOP/s, "
                  f"{r['GBps']:.0f} GB/s", flush=True)
        if want(which + "40"):
            r = bench_qlinear(torch, gdn, dev, timer, steps=max(10, args.steps // 8), warmup=3, which=which, M=40)
            sec[f"{which}_48_layers_m40"] = r
            print(f"# {which} x48 M=40 (4-bit, MFMA): {r['us_per_step']:.1f} us/step, {r['GBps']:.0f} GB/s, "
                  f"{r['TFLOPs']:.1f} TFLOP/s", flush=True)
    if "crossover" in only:
        sec["crossover_recurrent_vs_chunked"] = bench_crossover(torch, gdn, dev, timer, args.steps, 3)
    if want("copy"):
        cc = bench_copy_ceiling(torch, dev, timer)
        sec["copy_ceiling_GBps"] = round(cc["GBps"], 1)
        print(f"# device copy ceiling: {cc['GBps']:.0f} GB/s", flush=True)
        sc = stream_ceilings(torch, dev, timer, steps=max(20, args.steps // 2), b32="decode_b32_48_layers" in sec)
        if sc is not None:
            sec["stream_ceilings"] = sc
            if head is not None:
                best = max(sc["decode_shape_rmw_stream"]["GBps"], sc["decode_shape_rmw_stream_kheads"]["GBps"])
                sc["decode_vs_rmw_stream"] = round(head["GBps"] / best, 4)
                # time ratio of the decode step to the stream carrying the same 313.4 MB
                sc["decode_time_vs_full_bytes_stream"] = round(
                    sc["decode_full_bytes_rmw_stream"]["us"] / (head["ms_per_step"] * 1e3), 4)
            if "verify_b8_t5" in sec:
                sc["verify_vs_stream"] = round(sec["verify_b8_t5"]["GBps"] / sc["verify_shape_stream"]["GBps"], 4)
            if "decode_b32_shape_rmw_stream" in sc:
                best = max(sc["decode_b32_shape_rmw_stream"]["GBps"], sc["decode_b32_shape_rmw_stream_split"]["GBps"])
                sc["decode_b32_vs_rmw_stream"] = round(sec["decode_b32_48_layers"]["GBps"] / best, 4)
            print(f"# same-shape streams: decode RMW {sc['decode_shape_rmw_stream']['us']:.1f} us "
                  f"({sc['decode_shape_rmw_stream']['GBps']:.0f} GB/s; in the kernel's order "
                  f"{sc['decode_shape_rmw_stream_kheads']['us']:.1f} us; with the front end's bytes, 313.4 MB, "
                  f"{sc['decode_full_bytes_rmw_stream']['us']:.1f} us), read only "
                  f"{sc['decode_shape_read_stream']['GBps']:.0f} GB/s, write only "
                  f"{sc['decode_shape_write_stream']['GBps']:.0f} GB/s, verify "
                  f"{sc['verify_shape_stream']['us']:.1f} us ({sc['verify_shape_stream']['GBps']:.0f} GB/s)", flush=True)
            if "decode_b32_shape_rmw_stream" in sc:
                b, b2 = sc["decode_b32_shape_rmw_stream"], sc["decode_b32_shape_rmw_stream_split"]
                print(f"# same-shape streams: B=32 decode RMW {b['us'] / 1e3:.3f} ms ({b['GBps']:.0f} GB/s) in "
                      f"dispatch order, {b2['us'] / 1e3:.3f} ms ({b2['GBps']:.0f} GB/s) split per XCD", flush=True)

    if head is None:
        print(json.dumps({"secondary": sec}))
        return 0
    cpu = None if args.no_cpu else cpu_baseline()
    if cpu:
        print(f"# cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads", flush=True)
    # One launch per step: the back-to-back pass gives that launch's average duration
    # (dispatch gaps included, no timing packets between launches); the event-bracketed
    # per-launch durations are reported beside it.
    launch_us = head["ms_per_step"] * 1e3
    achieved = head["bytes_per_step"] / (launch_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(head["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "48-layer gated-delta decode step, B=1, conv front end + gates "
                               "+ recurrence (Hk=16, Hv=48, Dk=Dv=128, fp32 state)",
                   "layers": 48, "batch": 1, "seq_len": 1,
                   "state_sets_rotated": head["state_sets"],
                   "working_set_MB": round(head["working_set_MB"], 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": load_traffic("decode_b1_48_layers_conv"),
                     "kernel_us_avg": round(launch_us, 2),
                     "kernel_us_event_bracketed_avg": round(head["launch_ms_avg"] * 1e3, 2),
                     "kernel_us_event_bracketed_p10": round(head["launch_ms_p10"] * 1e3, 2),
                     "kernel_us_event_bracketed_p50": round(head["launch_ms_p50"] * 1e3, 2),
                     "kernel_us_event_bracketed_p90": round(head["launch_ms_p90"] * 1e3, 2),
                     "bytes_per_launch": head["bytes_per_step"]},
        "cpu_baseline": cpu,
        "secondary": sec,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
