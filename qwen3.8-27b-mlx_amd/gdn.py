"""Python host side of libgdn.so: ctypes bindings over the C ABI (include/gdn.h) and a
mirror of the reference's per-layer interface.

Mirrors (paths relative to the reference tree):
  run(...)              delta::run(q, k, v, alpha, beta, S, collect)   cpp/src/delta.hpp:66-68
                        (python: delta_kernel.gated_delta_metal, python/delta_kernel.py:126-165)
  layer(...)            the recurrent core of GatedDeltaNet::operator() from the conv input
                        to o: cpp/src/model.cpp:585-624 (gates 608-612)
  prefill_chunked(...)  chunked_delta, python/qwen35.py:365-431
  DeltaCache            DeltaCache + commit, cpp/src/model.hpp:211-227, model.cpp:439-457

Tensors are torch tensors on the GPU (torch supplies device memory and the stream;
the computation is the HIP library's). Errors from the library raise GdnError with the
library's message; nothing falls back to another implementation.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import List, Optional

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libgdn.so")

GDN_OK, GDN_EINVAL, GDN_EUNSUPPORTED, GDN_EDEVICE = 0, 1, 2, 3
DTYPE_BF16, DTYPE_F32 = 0, 1
FRONTEND_QKV, FRONTEND_CONV = 0, 1
GATES_RAW, GATES_PRECOMPUTED = 0, 1
PREFILL_ACCURATE, PREFILL_FAST = 0, 1  # gdn_prefill_precision; the first is the default
STATES_BHT, STATES_TBH = 0, 1
HEAD_DIM = 128
CONV_TAPS = 4

# Calls that do not record and carry at least chunked_min_t(B) tokens run the chunked form
# (gdn_prefill_chunked, the accurate precision); shorter ones the recurrent kernel (gdn_run),
# serial in T. Measured on MI355X with one layer and the conv front end (bench.py's
# crossover: recurrent against chunked, T = 24 .. 96): the chunked form takes 26.2-26.7 /
# 33.5-34.4 / 42.6-43.9 / 63.5-68.6 us at B = 1 / 2 / 4 / 8 up to T = 64; the recurrent kernel
# 23.2 / 26.4 / 27.6 us at B = 1 and T = 32 / 36 / 40, 32.2 / 33.8 / 38.8 us at B = 2 and
# T = 28 / 32 / 36, 42.7 / 46.5 us at B = 4 and T = 28 / 32, 59.3 / 64.8 / 74.1 us at B = 8
# and T = 28 / 32 / 36. The forms meet near T = 36, 32, 30 and 32 for B = 1, 2, 4 and 8.
# Module-level so that tests can force either form, as the reference's CHUNK_THRESHOLD
# (python/qwen35.py:338, 606-626), which makes the same choice by length.
CHUNKED_MIN_T = 28
_CHUNKED_MIN_T_BY_B = {1: 36, 2: 32, 3: 31, 4: 30}


def chunked_min_t(B: int) -> int:
    """Fewest tokens of a non-recording call of B sequences that run on the chunked form."""
    return max(CHUNKED_MIN_T, _CHUNKED_MIN_T_BY_B.get(B, 32))

QLINEAR_MAX_SEGS = 4
QLINEAR_GEMV_ROWS = 4
QLINEAR_MAX_ROWS = 4096
QLINEAR_NOALLOC_SCRATCH_BYTES = 9 << 20

EXPORTS = ("gdn_run", "gdn_prefill_chunked", "gdn_prefill_chunked_timed", "gdn_prefill_workspace_size", "gdn_commit",
           "gdn_qlinear", "gdn_qlinear_workspace_size", "gdn_qlinear_noalloc", "gdn_available",
           "gdn_abi_version", "gdn_last_error")


class GdnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[gdn error {code}] {msg}")
        self.code = code


_vp = ctypes.c_void_p
_int = ctypes.c_int


class LayerArgs(ctypes.Structure):
    """struct gdn_layer_args (include/gdn.h)."""
    _fields_ = [
        ("n_layers", _int), ("batch", _int), ("seq_len", _int), ("num_k_heads", _int),
        ("num_v_heads", _int),
        ("frontend", _int),
        ("q", _vp), ("k", _vp), ("v", _vp), ("qkv_dtype", _int),
        ("x", _vp), ("conv_weight", _vp), ("conv_state_in", _vp), ("conv_state_out", _vp),
        ("gate_mode", _int),
        ("a", _vp), ("b", _vp), ("A_log", _vp), ("dt_bias", _vp),
        ("alpha", _vp), ("beta", _vp),
        ("state_in", _vp), ("state_out", _vp), ("states", _vp), ("states_layout", _int),
        ("o", _vp), ("o_dtype", _int),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("stream", _vp),
        ("prefill_precision", _int),
    ]


class CommitArgs(ctypes.Structure):
    """struct gdn_commit_args (include/gdn.h)."""
    _fields_ = [
        ("n_layers", _int), ("batch", _int), ("seq_len", _int), ("num_v_heads", _int),
        ("conv_dim", _int), ("n", _int),
        ("states", _vp), ("states_layout", _int),
        ("state_prev", _vp), ("state_dst", _vp),
        ("conv_state_in", _vp), ("x", _vp), ("conv_state_dst", _vp),
        ("stream", _vp),
    ]


class QLinearSeg(ctypes.Structure):
    """struct gdn_qlinear_seg (include/gdn.h)."""
    _fields_ = [("w", _vp), ("scales", _vp), ("biases", _vp), ("y", _vp), ("n", _int)]


class QLinearArgs(ctypes.Structure):
    """struct gdn_qlinear_args (include/gdn.h)."""
    _fields_ = [
        ("n_layers", _int), ("m", _int), ("k", _int),
        ("x", _vp),
        ("norm_x", _vp), ("norm_z", _vp), ("norm_gamma", _vp), ("norm_eps", ctypes.c_float),
        ("n_segs", _int), ("segs", QLinearSeg * QLINEAR_MAX_SEGS),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("stream", _vp),
    ]


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libgdn.so from the package directory; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        L.gdn_run.argtypes = [ctypes.POINTER(LayerArgs)]
        L.gdn_run.restype = _int
        L.gdn_prefill_chunked.argtypes = [ctypes.POINTER(LayerArgs)]
        L.gdn_prefill_chunked.restype = _int
        L.gdn_prefill_chunked_timed.argtypes = [ctypes.POINTER(LayerArgs), ctypes.POINTER(ctypes.c_float)]
        L.gdn_prefill_chunked_timed.restype = _int
        L.gdn_prefill_workspace_size.argtypes = [ctypes.POINTER(LayerArgs), ctypes.POINTER(ctypes.c_size_t)]
        L.gdn_prefill_workspace_size.restype = _int
        L.gdn_commit.argtypes = [ctypes.POINTER(CommitArgs)]
        L.gdn_commit.restype = _int
        L.gdn_qlinear.argtypes = [ctypes.POINTER(QLinearArgs)]
        L.gdn_qlinear.restype = _int
        L.gdn_qlinear_workspace_size.argtypes = [ctypes.POINTER(QLinearArgs), ctypes.POINTER(ctypes.c_size_t)]
        L.gdn_qlinear_workspace_size.restype = _int
        L.gdn_qlinear_noalloc.argtypes = [ctypes.POINTER(QLinearArgs)]
        L.gdn_qlinear_noalloc.restype = _int
        L.gdn_available.argtypes = []
        L.gdn_available.restype = _int
        L.gdn_abi_version.argtypes = []
        L.gdn_abi_version.restype = _int
        L.gdn_last_error.argtypes = []
        L.gdn_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def last_error() -> str:
    return lib().gdn_last_error().decode()


def available() -> bool:
    """delta::available (cpp/src/delta.cpp:133-135): a gfx950 device is current."""
    return bool(lib().gdn_available())


def _check(rc: int) -> None:
    if rc != GDN_OK:
        raise GdnError(rc, last_error())


def call_run(args: LayerArgs) -> None:
    _check(lib().gdn_run(ctypes.byref(args)))


def call_prefill(args: LayerArgs) -> None:
    _check(lib().gdn_prefill_chunked(ctypes.byref(args)))


def call_prefill_timed(args: LayerArgs) -> tuple:
    """gdn_prefill_chunked_timed: runs the chunked prefill, waits for it and returns the
    durations (ms) of its front-end, intra-chunk and scan kernels."""
    ms = (ctypes.c_float * 3)()
    _check(lib().gdn_prefill_chunked_timed(ctypes.byref(args), ms))
    return tuple(ms)


def call_commit(args: CommitArgs) -> None:
    _check(lib().gdn_commit(ctypes.byref(args)))


def call_qlinear(args: QLinearArgs) -> None:
    _check(lib().gdn_qlinear(ctypes.byref(args)))


def call_qlinear_noalloc(args: QLinearArgs) -> None:
    _check(lib().gdn_qlinear_noalloc(ctypes.byref(args)))


def qlinear_workspace_size(m: int, k: int, n_layers: int = 1) -> int:
    """Workspace bytes gdn_qlinear needs for m operand rows of k (0 on the GEMV path)."""
    a = QLinearArgs(n_layers=n_layers, m=m, k=k)
    n = ctypes.c_size_t(0)
    _check(lib().gdn_qlinear_workspace_size(ctypes.byref(a), ctypes.byref(n)))
    return n.value


def prefill_workspace_size(B: int, T: int, Hk: int = 16, Hv: int = 48, conv: bool = True,
                           precision: int = PREFILL_ACCURATE) -> int:
    """Workspace bytes of gdn_prefill_chunked; `conv` for the conv front end (x given),
    `precision` a PREFILL_* value."""
    args = LayerArgs(n_layers=1, batch=B, seq_len=T, num_k_heads=Hk, num_v_heads=Hv,
                     frontend=FRONTEND_CONV if conv else FRONTEND_QKV, prefill_precision=precision)
    out = ctypes.c_size_t(0)
    _check(lib().gdn_prefill_workspace_size(ctypes.byref(args), ctypes.byref(out)))
    return out.value


# --------------------------------------------------------------------------
# torch-facing helpers

def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if not t.is_contiguous():
        raise GdnError(GDN_EINVAL, "tensors passed to libgdn must be contiguous")
    return t.data_ptr()


def _dt(t) -> int:
    import torch
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise GdnError(GDN_EINVAL, f"unsupported dtype {t.dtype}")


def _stream(stream) -> Optional[int]:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


@dataclass
class Result:
    """delta::Result (cpp/src/delta.hpp:53-57)."""
    o: object
    s_out: object
    states: List[object] = field(default_factory=list)


def run(q, k, v, alpha, beta, S=None, collect: bool = False, *, o_dtype=None, stream=None,
        in_place: bool = False) -> Result:
    """delta::run: q, k (B,L,H,128) head-expanded; v (B,L,H,128); alpha, beta (B,L,H) fp32;
    S (B,H,128,128) fp32 or None. Returns o (B,L,H,128), s_out, and with collect the L
    per-step states as views of one (B,H,L,128,128) buffer (delta.cpp:155-171)."""
    import torch
    B, L, H, _ = q.shape
    o_dtype = torch.float32 if o_dtype is None else o_dtype
    o = torch.empty((B, L, H, HEAD_DIM), dtype=o_dtype, device=q.device)
    if in_place:
        if S is None:
            raise GdnError(GDN_EINVAL, "in-place run needs a state")
        s_out = S
    else:
        s_out = torch.empty((B, H, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=q.device)
    S_all = (torch.empty((B, H, L, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=q.device)
             if collect else None)
    args = LayerArgs(
        n_layers=1, batch=B, seq_len=L, num_k_heads=q.shape[2], num_v_heads=v.shape[2],
        frontend=FRONTEND_QKV, q=_ptr(q), k=_ptr(k), v=_ptr(v), qkv_dtype=_dt(q),
        gate_mode=GATES_PRECOMPUTED, alpha=_ptr(alpha), beta=_ptr(beta),
        state_in=_ptr(S), state_out=_ptr(s_out), states=_ptr(S_all), states_layout=STATES_BHT,
        o=_ptr(o), o_dtype=_dt(o), stream=_stream(stream))
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise GdnError(GDN_EINVAL, "q, k, v must share a dtype")
    call_run(args)
    states = [S_all[:, :, t] for t in range(L)] if collect else []
    return Result(o, s_out, states)


def layer_args(*, B: int, T: int, Hk: int = 16, Hv: int = 48, n_layers: int = 1,
               q=None, k=None, v=None, x=None, conv_weight=None, conv_state_in=None,
               conv_state_out=None, a=None, b=None, A_log=None, dt_bias=None, alpha=None,
               beta=None, state_in=None, state_out=None, states=None,
               states_layout: int = STATES_BHT, o=None, workspace=None,
               stream=None, precision: int = PREFILL_ACCURATE) -> LayerArgs:
    """Fill gdn_layer_args from torch tensors (front end and gate mode inferred)."""
    conv = x is not None
    raw = a is not None
    return LayerArgs(
        n_layers=n_layers, batch=B, seq_len=T, num_k_heads=Hk, num_v_heads=Hv,
        frontend=FRONTEND_CONV if conv else FRONTEND_QKV,
        q=_ptr(q), k=_ptr(k), v=_ptr(v), qkv_dtype=_dt(q) if q is not None else DTYPE_BF16,
        x=_ptr(x), conv_weight=_ptr(conv_weight), conv_state_in=_ptr(conv_state_in),
        conv_state_out=_ptr(conv_state_out),
        gate_mode=GATES_RAW if raw else GATES_PRECOMPUTED,
        a=_ptr(a), b=_ptr(b), A_log=_ptr(A_log), dt_bias=_ptr(dt_bias),
        alpha=_ptr(alpha), beta=_ptr(beta),
        state_in=_ptr(state_in), state_out=_ptr(state_out), states=_ptr(states),
        states_layout=states_layout,
        o=_ptr(o), o_dtype=_dt(o) if o is not None else DTYPE_BF16,
        workspace=_ptr(workspace),
        workspace_bytes=0 if workspace is None else workspace.numel() * workspace.element_size(),
        stream=_stream(stream), prefill_precision=precision)


def _use_chunked(B: int, T: int, record: bool, x, q, tensors) -> bool:
    """The length-based choice of the form (chunked_min_t), for calls the chunked form takes:
    not recording, bf16 q, k, v when given, 16-byte aligned inputs."""
    import torch
    if record or T < chunked_min_t(B):
        return False
    if x is None and q.dtype != torch.bfloat16:
        return False
    return all(t is None or t.data_ptr() % 16 == 0 for t in tensors)


def layer(*, x=None, q=None, k=None, v=None, a, b, A_log, dt_bias, state=None,
          conv_weight=None, conv_state=None, collect: bool = False, in_place: bool = True,
          o_dtype=None, Hk: int = 16, workspace=None, stream=None, precision: int = PREFILL_ACCURATE):
    """The per-layer call of GatedDeltaNet::operator() (cpp/src/model.cpp:585-641) at the
    recurrence: (q,k,v | x,conv) + (a,b,A_log,dt_bias) + state ->
    (o, state'). x is (B,T,C) bf16 for the conv front end; otherwise q,k (B,T,Hk,128),
    v (B,T,Hv,128). Returns dict(o, state, states, conv_state). A call that does not record
    and has at least chunked_min_t(B) tokens runs the chunked form (python/qwen35.py:606-626)
    in `workspace` (uint8, at least prefill_workspace_size(B, T, ...) bytes), which is
    allocated here only when the caller gives none.

    Precision (`precision`, PREFILL_*): PREFILL_ACCURATE, the default, carries the state
    products at fp32 accuracy (V' = T' (V - e^G K S) with S, X = V - e^G K S and T' split
    into bf16 hi + lo, V'' split in K^T V''), as the reference's fp32 Metal kernel for every
    window (cpp/src/model.cpp:619-624): the state ends within about 1e-5 (relative) of the
    fp32 recurrence whatever the gates. PREFILL_FAST (bf16 operands, X alone split) leaves
    it about 2e-3 to 4e-3 off in about 0.85 of the time. The recurrent kernel is within about
    1e-7.
    Later decode steps continue from that state."""
    import torch
    src = x if x is not None else q
    B, T = src.shape[0], src.shape[1]
    Hv = A_log.shape[-1]
    dev = src.device
    o = torch.empty((B, T, Hv, HEAD_DIM), dtype=o_dtype or torch.bfloat16, device=dev)
    record = collect
    if record:
        state_out = None
    elif in_place and state is not None:
        state_out = state
    else:
        state_out = torch.empty((B, Hv, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev)
    states = (torch.empty((B, Hv, T, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev)
              if record else None)
    conv_out = None
    if x is not None and not record:
        conv_out = torch.empty((B, CONV_TAPS - 1, x.shape[2]), dtype=torch.bfloat16, device=dev)
    chunked = _use_chunked(B, T, record, x, q, (x, conv_state, q, k, v))
    ws = None
    if chunked:
        ws = workspace if workspace is not None else torch.empty(
            prefill_workspace_size(B, T, Hk, Hv, conv=x is not None, precision=precision), dtype=torch.uint8,
            device=dev)
    args = layer_args(B=B, T=T, Hk=Hk, Hv=Hv, q=q, k=k, v=v, x=x, conv_weight=conv_weight,
                      conv_state_in=conv_state, conv_state_out=conv_out, a=a, b=b,
                      A_log=A_log, dt_bias=dt_bias, state_in=state, state_out=state_out,
                      states=states, o=o, workspace=ws, stream=stream, precision=precision)
    (call_prefill if chunked else call_run)(args)
    return dict(o=o, state=state_out, states=states, conv_state=conv_out)


def prefill_chunked(*, x=None, q=None, k=None, v=None, a=None, b=None, A_log=None,
                    dt_bias=None, alpha=None, beta=None, state=None, conv_weight=None,
                    conv_state=None, o_dtype=None, Hk: int = 16, Hv: int = 48, workspace=None,
                    stream=None, precision: int = PREFILL_ACCURATE):
    """chunked_delta (python/qwen35.py:365-431) with the conv front end and gates inside.
    Returns dict(o, state, conv_state). The workspace is allocated here unless given;
    `precision` is a PREFILL_* value (see layer())."""
    import torch
    src = x if x is not None else q
    B, T = src.shape[0], src.shape[1]
    dev = src.device
    o = torch.empty((B, T, Hv, HEAD_DIM), dtype=o_dtype or torch.bfloat16, device=dev)
    state_out = torch.empty((B, Hv, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev)
    conv_out = (torch.empty((B, CONV_TAPS - 1, x.shape[2]), dtype=torch.bfloat16, device=dev)
                if x is not None else None)
    if workspace is None and T > 0:
        workspace = torch.empty(prefill_workspace_size(B, T, Hk, Hv, conv=x is not None, precision=precision),
                                dtype=torch.uint8, device=dev)
    args = layer_args(B=B, T=T, Hk=Hk, Hv=Hv, q=q, k=k, v=v, x=x, conv_weight=conv_weight,
                      conv_state_in=conv_state, conv_state_out=conv_out, a=a, b=b,
                      A_log=A_log, dt_bias=dt_bias, alpha=alpha, beta=beta, state_in=state,
                      state_out=state_out, o=o, workspace=workspace, stream=stream, precision=precision)
    call_prefill(args)
    return dict(o=o, state=state_out, conv_state=conv_out)


def commit(*, n: int, T: int, states, state_prev, state_dst, x=None, conv_state_in=None,
           conv_state_dst=None, states_layout: int = STATES_BHT, n_layers: int = 1,
           stream=None) -> None:
    """DeltaCache::commit(n) on the device (cpp/src/model.cpp:439-457)."""
    B, Hv = state_dst.shape[-4], state_dst.shape[-3]
    C = x.shape[-1] if x is not None else (conv_state_dst.shape[-1] if conv_state_dst is not None else 0)
    args = CommitArgs(n_layers=n_layers, batch=B, seq_len=T, num_v_heads=Hv, conv_dim=C, n=n,
                      states=_ptr(states), states_layout=states_layout,
                      state_prev=_ptr(state_prev), state_dst=_ptr(state_dst),
                      conv_state_in=_ptr(conv_state_in), x=_ptr(x),
                      conv_state_dst=_ptr(conv_state_dst), stream=_stream(stream))
    call_commit(args)


class DeltaCache:
    """DeltaCache (cpp/src/model.hpp:211-227) over device buffers: `record` mode keeps
    the per-step states of a block instead of advancing; commit(n) adopts step n.

    The per-step states of a block are recorded in (T, B, Hv) order, so step n-1 is one
    contiguous state and commit(n) adopts it by pointer: `state` becomes a view of the
    recorded block and no state is copied (only the 3-row conv window moves).

    The conv state is kept in two buffers that swap roles each call (the library never
    updates it in place: every workgroup must see the old rows).

    Blocks of chunked_min_t(B) .. max_prefill_tokens tokens that are not recorded run the
    chunked form in a workspace allocated here, once (the reference prefills in windows of
    1024, cpp/src/session.hpp:136); max_prefill_tokens = 0 keeps every block on the
    recurrent kernel. As the C++ DeltaCache (include/gdn.hpp), step() then allocates no
    workspace. `prefill_precision` is PREFILL_ACCURATE (the default) or PREFILL_FAST (see
    layer()); the recurrent kernel stays within about 1e-7 of the fp32 recurrence."""

    def __init__(self, B: int, Hv: int = 48, Hk: int = 16, device="cuda", max_prefill_tokens: int = 0,
                 prefill_precision: int = PREFILL_ACCURATE):
        import torch
        C = 2 * Hk * HEAD_DIM + Hv * HEAD_DIM
        self.Hk, self.Hv, self.C = Hk, Hv, C
        self.state = torch.zeros((B, Hv, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=device)
        self.conv = torch.zeros((B, CONV_TAPS - 1, C), dtype=torch.bfloat16, device=device)
        self._conv_spare = torch.empty_like(self.conv)
        self.max_prefill_tokens = max_prefill_tokens if max_prefill_tokens >= chunked_min_t(B) else 0
        self.prefill_precision = prefill_precision
        self._ws = (torch.empty(prefill_workspace_size(B, self.max_prefill_tokens, Hk, Hv,
                                                       precision=prefill_precision),
                                dtype=torch.uint8, device=device) if self.max_prefill_tokens else None)
        self.offset = 0
        self.record = False
        self.base_offset = 0
        self.pending = None

    def step(self, x, conv_weight, a, b, A_log, dt_bias, o_dtype=None, stream=None):
        """One GatedDeltaNet recurrence call (model.cpp:585-638) on this cache; a block of
        chunked_min_t(B) .. max_prefill_tokens tokens that is not recorded runs the chunked
        form in the cache's workspace."""
        import torch
        B, T = x.shape[0], x.shape[1]
        o = torch.empty((B, T, self.Hv, HEAD_DIM), dtype=o_dtype or torch.bfloat16,
                        device=x.device)
        if self.record:
            states = torch.empty((T, B, self.Hv, HEAD_DIM, HEAD_DIM), dtype=torch.float32,
                                 device=x.device)
            args = layer_args(B=B, T=T, Hk=self.Hk, Hv=self.Hv, x=x, conv_weight=conv_weight,
                              conv_state_in=self.conv, a=a, b=b, A_log=A_log, dt_bias=dt_bias,
                              state_in=self.state, states=states, states_layout=STATES_TBH,
                              o=o, stream=stream)
            call_run(args)
            self.base_offset = self.offset
            self.pending = (x, states, T)
        else:
            chunked = (self._ws is not None and T <= self.max_prefill_tokens
                       and _use_chunked(B, T, False, x, None, (x, o)))
            args = layer_args(B=B, T=T, Hk=self.Hk, Hv=self.Hv, x=x, conv_weight=conv_weight,
                              conv_state_in=self.conv, conv_state_out=self._conv_spare, a=a,
                              b=b, A_log=A_log, dt_bias=dt_bias, state_in=self.state,
                              state_out=self.state, o=o, workspace=self._ws if chunked else None,
                              stream=stream, precision=self.prefill_precision)
            (call_prefill if chunked else call_run)(args)
            self.conv, self._conv_spare = self._conv_spare, self.conv
            self.offset += T
        return o

    def commit(self, n: int, stream=None) -> None:
        """Accept the first n tokens of the recorded block (model.cpp:439-457)."""
        if self.pending is None:
            return
        x, states, T = self.pending
        if n < 0 or n > T:
            raise GdnError(GDN_EINVAL, "DeltaCache::commit out of range")
        adopted = self.state if n == 0 else states[n - 1]   # the pointer swap
        commit(n=n, T=T, states=states, state_prev=self.state, state_dst=adopted, x=x,
               conv_state_in=self.conv, conv_state_dst=self.conv, states_layout=STATES_TBH,
               stream=stream)
        self.state = adopted
        self.offset = self.base_offset + n
        self.pending = None
        self.record = False


# --------------------------------------------------------------------------
# quantized linear: Linear::operator() for 4-bit weights (cpp/src/model.cpp:356-372)

@dataclass
class QuantLinear:
    """One quantized weight as the reference stores it (cpp/src/model.hpp Linear): w
    (N, K/8) uint32 (stored as int32 by torch), scales and biases (N, K/64) bf16; with a
    leading layer dimension when several layers are stacked."""
    w: object
    scales: object
    biases: object

    @property
    def n(self) -> int:
        return self.w.shape[-2]


def qlinear_args(mats, x=None, *, norm=None, n_layers: int = 1, workspace=None, stream=None,
                 alloc_workspace: bool = True):
    """gdn_qlinear_args for y_i = x W_i^T, i over `mats` (1..4 QuantLinear reading the same
    x), or with norm = (o, z, gamma, eps) the layer's GatedRMSNorm of o as the operand.
    Allocates the outputs, and (with alloc_workspace) the workspace when the rows need one
    and none is given; returns (args, [y_i])."""
    import torch
    src = x if x is not None else norm[0]
    K = src.shape[-1]
    M = src.shape[-2]
    ys = []
    a = QLinearArgs(n_layers=n_layers, m=M, k=K, x=_ptr(x), n_segs=len(mats), stream=_stream(stream))
    if norm is not None:
        o, z, gamma, eps = norm
        a.norm_x, a.norm_z, a.norm_gamma, a.norm_eps = _ptr(o), _ptr(z), _ptr(gamma), float(eps)
    for i, q in enumerate(mats):
        shape = (n_layers, M, q.n) if n_layers > 1 else (M, q.n)
        y = torch.empty(shape, dtype=torch.bfloat16, device=src.device)
        ys.append(y)
        a.segs[i] = QLinearSeg(w=_ptr(q.w), scales=_ptr(q.scales), biases=_ptr(q.biases), y=_ptr(y), n=q.n)
    try:
        need = qlinear_workspace_size(M, K, n_layers)
    except GdnError:
        need = 0  # a bad shape: gdn_qlinear itself reports it
    if need and workspace is None and alloc_workspace:
        workspace = torch.empty(need, dtype=torch.uint8, device=src.device)
    if workspace is not None:
        a.workspace = _ptr(workspace)
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    a._keep = workspace  # the workspace lives as long as the args
    return a, ys


def qlinear(mats, x=None, *, norm=None, n_layers: int = 1, workspace=None, stream=None):
    """Linear::operator() for quantized weights (model.cpp:356-372) over 1..4 matrices
    sharing x -- e.g. the layer's in_proj_qkv, in_proj_z, in_proj_a, in_proj_b -- or, with
    norm = (o, z, gamma, eps), out_proj(GatedRMSNorm(o, z)) (model.cpp:626-641). Up to
    QLINEAR_GEMV_ROWS rows it is the GEMV kernel; more rows run on MFMA with a workspace
    (allocated here unless given)."""
    args, ys = qlinear_args(mats, x, norm=norm, n_layers=n_layers, workspace=workspace, stream=stream)
    call_qlinear(args)
    return ys


def qlinear_noalloc(mats, x=None, *, norm=None, n_layers: int = 1, stream=None):
    """qlinear through gdn_qlinear_noalloc: no workspace, the library's per-device scratch
    of 9 MiB instead -- 512 operand rows at any k, 1,024 rows up to k = 4096; larger shapes
    return GDN_EINVAL (e.g. M = 4096 at K = 5120 needs 41.25 MiB). Calls overlapping on one
    device race on the scratch. Only the outputs are allocated here; the library call itself
    allocates nothing."""
    args, ys = qlinear_args(mats, x, norm=norm, n_layers=n_layers, stream=stream, alloc_workspace=False)
    call_qlinear_noalloc(args)
    return ys
