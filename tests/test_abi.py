"""CPU tests of the C ABI (include/gdn.h): the library loads, exports every declared
symbol, its ctypes mirror matches the C struct layout, and argument errors come back as
GDN_EINVAL with a message before any device work -- no GPU is needed for any of it."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gdn.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|size_t)\s+(gdn_\w+)\s*\(", text, re.M)))


def test_header_declares_the_entry_points():
    assert declared_functions() == sorted(
        ["gdn_run", "gdn_prefill_chunked", "gdn_prefill_chunked_timed", "gdn_prefill_workspace_size", "gdn_commit",
         "gdn_qlinear", "gdn_qlinear_workspace_size", "gdn_qlinear_noalloc", "gdn_available",
         "gdn_abi_version", "gdn_last_error"])


def test_library_exports_every_declared_symbol(gdn):
    L = gdn.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", gdn.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(gdn_\w+)", out))
    assert set(declared_functions()) <= exported
    assert L.gdn_abi_version() == 5
    assert set(gdn.EXPORTS) == set(declared_functions())


def _c_layout(struct: str, fields):
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"gdn.h\"\nint main(void){\n"
    src += f'printf("%zu\\n", sizeof({struct}));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof({struct}, {f}));\n'
    src += "return 0;}\n"
    tmp = os.path.join("/tmp", f"gdn_layout_{os.getpid()}_{struct}")
    with open(tmp + ".c", "w") as fh:
        fh.write(src)
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), tmp + ".c", "-o",
                    tmp], check=True)
    out = subprocess.run([tmp], capture_output=True, text=True, check=True).stdout.split()
    os.remove(tmp)
    os.remove(tmp + ".c")
    return [int(x) for x in out]


@pytest.mark.parametrize("cls,struct", [("LayerArgs", "gdn_layer_args"),
                                        ("CommitArgs", "gdn_commit_args"),
                                        ("QLinearArgs", "gdn_qlinear_args"),
                                        ("QLinearSeg", "gdn_qlinear_seg")])
def test_ctypes_mirror_matches_c_layout(gdn, cls, struct):
    C = getattr(gdn, cls)
    names = [f for f, _ in C._fields_]
    layout = _c_layout(struct, names)
    assert layout[0] == ctypes.sizeof(C)
    assert layout[1:] == [getattr(C, n).offset for n in names]


def _no_gpu():
    import torch
    return not torch.cuda.is_available()


def _args(gdn, **kw):
    base = dict(n_layers=1, batch=1, seq_len=1, num_k_heads=16, num_v_heads=48,
                frontend=gdn.FRONTEND_QKV, q=0x1000, k=0x2000, v=0x3000,
                qkv_dtype=gdn.DTYPE_BF16, gate_mode=gdn.GATES_RAW, a=0x4000, b=0x5000,
                A_log=0x6000, dt_bias=0x7000, state_in=0x100000, state_out=0x100000,
                o=0x9000000, o_dtype=gdn.DTYPE_BF16)
    base.update(kw)
    return gdn.LayerArgs(**base)


BAD_RUN = [
    (dict(n_layers=0), "n_layers"),
    (dict(batch=-1), "batch"),
    (dict(seq_len=-2), "seq_len"),
    (dict(num_k_heads=0), "head counts"),
    (dict(num_v_heads=40), "multiple"),
    (dict(frontend=7), "frontend"),
    (dict(gate_mode=3), "gate_mode"),
    (dict(o_dtype=9), "o_dtype"),
    (dict(qkv_dtype=4), "qkv_dtype"),
    (dict(states_layout=2), "states_layout"),
    (dict(q=None), "q, k and v"),
    (dict(a=None), "raw gates"),
    (dict(gate_mode=1), "precomputed"),
    (dict(o=None), "o is required"),
    (dict(state_in=0x100004), "16-byte"),
    (dict(state_out=0x100000 + 4096), "state_out must equal"),
    (dict(states=0x100000 + 64), "states must not overlap state_in"),
    (dict(o=0x100000 + 128), "o must not overlap"),
    (dict(frontend=1, x=None, conv_weight=0x8000), "x is required"),
    (dict(frontend=1, x=0xA000000, conv_weight=None), "conv_weight"),
    (dict(frontend=1, x=0xA000000, conv_weight=0x8000, conv_state_in=0xB000000,
          conv_state_out=0xB000000 + 2), "conv_state_out must not overlap conv_state_in"),
    (dict(frontend=1, x=0xA000000, conv_weight=0x8000, conv_state_out=0xA000000),
     "must not overlap x"),
    (dict(n_layers=48, batch=1 << 20), "too large"),
]


@pytest.mark.parametrize("kw,msg", BAD_RUN)
def test_run_rejects_bad_arguments(gdn, kw, msg):
    L = gdn.lib()
    rc = L.gdn_run(ctypes.byref(_args(gdn, **kw)))
    assert rc == gdn.GDN_EINVAL
    assert msg in gdn.last_error(), gdn.last_error()


def test_prefill_workspace_size_and_checks(gdn):
    # per chunk: Q, K and K^T per k-head (bf16 64 x 128); V in fragment order (bf16) and T'
    # hi/lo per v-head; two pairs of gate factors per position; 256-byte aligned pieces. The
    # same for both precisions (the fast one leaves the T' lo blocks unused) and front ends.
    n_qkv = gdn.prefill_workspace_size(1, 4096, conv=False)
    assert n_qkv == 3 * 16 * 64 * 8192 * 2 + 2 * 48 * 64 * 8192 * 2 + 2 * 48 * 64 * 128 * 4
    assert gdn.prefill_workspace_size(1, 4096) == n_qkv
    # a ragged T: whole chunks for the per-chunk pieces
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    nc = (100 + 63) // 64
    assert gdn.prefill_workspace_size(2, 100) == (
        3 * al(2 * 16 * nc * 8192 * 2) + 2 * al(2 * 48 * nc * 8192 * 2) + 2 * al(2 * 48 * nc * 128 * 4))
    assert gdn.PREFILL_ACCURATE == 0   # a zeroed gdn_layer_args gets the accurate form
    for conv in (True, False):
        for T in (4096, 100, 1):
            assert gdn.prefill_workspace_size(2, T, conv=conv, precision=gdn.PREFILL_FAST) == (
                gdn.prefill_workspace_size(2, T, conv=conv))
    with pytest.raises(gdn.GdnError, match="prefill_precision"):
        gdn.prefill_workspace_size(1, 64, precision=2)
    L = gdn.lib()
    rc = L.gdn_prefill_chunked(ctypes.byref(_args(gdn, seq_len=100)))
    assert rc == gdn.GDN_EINVAL and "workspace" in gdn.last_error()
    rc = L.gdn_prefill_chunked(ctypes.byref(_args(gdn, seq_len=100, prefill_precision=7)))
    assert rc == gdn.GDN_EINVAL and "prefill_precision" in gdn.last_error()
    rc = L.gdn_prefill_chunked(ctypes.byref(_args(gdn, seq_len=100, qkv_dtype=gdn.DTYPE_F32)))
    assert rc == gdn.GDN_EINVAL and "bf16" in gdn.last_error()
    rc = L.gdn_prefill_chunked(ctypes.byref(_args(gdn, seq_len=100, workspace=0x10000010,
                                                  workspace_bytes=1 << 40)))
    assert rc == gdn.GDN_EINVAL and "256-byte" in gdn.last_error()
    # the outputs are written as 16-byte pieces of a position's columns
    rc = L.gdn_prefill_chunked(ctypes.byref(_args(gdn, seq_len=100, o=0x9000002, workspace=0x10000000,
                                                  workspace_bytes=1 << 40)))
    assert rc == gdn.GDN_EINVAL and "o must be 16-byte aligned" in gdn.last_error()


@pytest.mark.parametrize("kw,name", [
    (dict(o=0x10000000 + 4096), "o"),
    (dict(state_in=0x10000000 + 4096, state_out=0x10000000 + 4096), "state_in"),
    (dict(state_out=0x10000000 - 4096), "state_out"),   # ends inside the workspace
    (dict(a=0x10000000 + 256), "a"),
    (dict(A_log=0x10000000 + 512), "A_log"),
    (dict(v=0x10000000 - 256), "v"),
    (dict(frontend=1, x=0x10000000 + 4096, conv_weight=0x8000), "x"),
    (dict(frontend=1, x=0xA000000, conv_weight=0x8000, conv_state_out=0x10000000), "conv_state_out"),
    (dict(gate_mode=1, a=None, b=None, alpha=0x8000000, beta=0x10000000 + 1024), "beta"),
])
def test_prefill_rejects_a_workspace_that_overlaps(gdn, kw, name):
    """The workspace is written while every other buffer is live: any overlap is an error."""
    base = dict(seq_len=100, workspace=0x10000000, workspace_bytes=1 << 28)
    base.update(kw)
    rc = gdn.lib().gdn_prefill_chunked(ctypes.byref(_args(gdn, **base)))
    assert rc == gdn.GDN_EINVAL, gdn.last_error()
    assert f"the workspace must not overlap {name}" in gdn.last_error(), gdn.last_error()


def test_null_args_and_prefill_states(gdn):
    L = gdn.lib()
    assert L.gdn_run(None) == gdn.GDN_EINVAL and "NULL" in gdn.last_error()
    assert L.gdn_prefill_chunked(None) == gdn.GDN_EINVAL
    ms = (ctypes.c_float * 3)(1.0, 1.0, 1.0)
    assert L.gdn_prefill_chunked_timed(None, ms) == gdn.GDN_EINVAL and list(ms) == [0.0, 0.0, 0.0]
    assert L.gdn_prefill_chunked_timed(ctypes.byref(_args(gdn, seq_len=100)), None) == gdn.GDN_EINVAL
    assert "kernel_ms" in gdn.last_error()
    # the timed form checks its arguments as the plain one does, before any HIP call
    rc = L.gdn_prefill_chunked_timed(ctypes.byref(_args(gdn, seq_len=100)), ms)
    assert rc == gdn.GDN_EINVAL and "workspace" in gdn.last_error(), gdn.last_error()
    assert L.gdn_commit(None) == gdn.GDN_EINVAL
    rc = L.gdn_prefill_chunked(ctypes.byref(_args(gdn, states=0x9000000 * 4)))
    assert rc == gdn.GDN_EINVAL and "per-step states" in gdn.last_error()


def _commit(gdn, **kw):
    base = dict(n_layers=1, batch=1, seq_len=5, num_v_heads=48, conv_dim=10240, n=2,
                states=0x1000000, states_layout=gdn.STATES_BHT, state_prev=0x100000,
                state_dst=0x100000, conv_state_in=0x2000, x=0x40000000, conv_state_dst=0x2000)
    base.update(kw)
    return gdn.CommitArgs(**base)


@pytest.mark.parametrize("kw,msg", [
    (dict(n=6), "out of range"),
    (dict(n=-1), "out of range"),
    (dict(states_layout=5), "states_layout"),
    (dict(n=0, state_prev=None), "state_prev"),
    (dict(states=None), "states is required"),
    (dict(state_dst=None), "state_dst"),
    (dict(state_dst=0x1000000 + 4096), "overlaps states"),
    (dict(conv_state_dst=0x40000000 + 64), "must not overlap x"),
    (dict(x=None), "x is required"),
])
def test_commit_rejects_bad_arguments(gdn, kw, msg):
    rc = gdn.lib().gdn_commit(ctypes.byref(_commit(gdn, **kw)))
    assert rc == gdn.GDN_EINVAL
    assert msg in gdn.last_error(), gdn.last_error()


def test_empty_batch_is_a_no_op(gdn):
    # B = 0 touches nothing and needs no device
    assert gdn.lib().gdn_run(ctypes.byref(_args(gdn, batch=0))) == gdn.GDN_OK
    assert gdn.last_error() == ""


@pytest.mark.skipif(not _no_gpu(), reason="checks the no-device path")
def test_valid_call_without_device_reports_device_error(gdn):
    assert gdn.lib().gdn_available() == 0
    rc = gdn.lib().gdn_run(ctypes.byref(_args(gdn)))
    assert rc in (gdn.GDN_EDEVICE, gdn.GDN_EUNSUPPORTED)
    assert gdn.last_error()


def test_error_message_is_per_thread(gdn):
    import threading
    L = gdn.lib()
    L.gdn_run(ctypes.byref(_args(gdn, n_layers=0)))
    seen = {}

    def worker():
        seen["before"] = gdn.last_error()
        L.gdn_run(ctypes.byref(_args(gdn, batch=-1)))
        seen["after"] = gdn.last_error()

    th = threading.Thread(target=worker)
    th.start()
    th.join()
    assert seen["before"] == "" and "batch" in seen["after"]
    assert "n_layers" in gdn.last_error()


def test_product_does_not_touch_the_oracle():
    pkg = os.path.join(ROOT, "qwen3.8-27b-mlx_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h", ".hpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower() and "gdno_" not in text, f


def _ql(gdn, **kw):
    segs = kw.pop("segs", None)
    base = dict(n_layers=1, m=1, k=5120, x=0x10000, n_segs=1)
    base.update(kw)
    a = gdn.QLinearArgs(**base)
    for i, sg in enumerate(segs or [dict(w=0x1000000, scales=0x2000000, biases=0x3000000, y=0x4000000, n=64)]):
        a.segs[i] = gdn.QLinearSeg(**sg)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(m=0), "bad shape"),
    (dict(m=4097), "bad shape"),
    (dict(n_layers=0), "bad shape"),
    (dict(k=5000), "unsupported"),
    (dict(m=5), "needs a workspace"),
    (dict(m=4, k=8192), "needs a workspace"),
    (dict(m=40, workspace=0x8000000, workspace_bytes=100), "needs a workspace"),
    (dict(m=40, workspace=0x8000010, workspace_bytes=1 << 30), "256-byte"),
    (dict(m=40, workspace=0x10000, workspace_bytes=1 << 30), "must not overlap the operand"),
    (dict(m=40, workspace=0x3ffff00, workspace_bytes=1 << 20), "must not overlap the workspace"),
    (dict(n_segs=5), "n_segs"),
    (dict(x=None), "exactly one"),
    (dict(norm_x=0x20000), "exactly one"),
    (dict(x=None, norm_x=0x20000), "norm_z and norm_gamma"),
    (dict(x=0x10008), "16-byte"),
    (dict(segs=[dict(w=0x1000000, scales=0x2000000, biases=0, y=0x4000000, n=64)]), "segment 0"),
    (dict(segs=[dict(w=0x1000008, scales=0x2000000, biases=0x3000000, y=0x4000000, n=64)]), "16-byte"),
    (dict(segs=[dict(w=0x1000000, scales=0x2000004, biases=0x3000000, y=0x4000000, n=64)]), "8-byte"),
    (dict(segs=[dict(w=0x1000000, scales=0x2000000, biases=0x3000002, y=0x4000000, n=64)]), "8-byte"),
    (dict(segs=[dict(w=0x1000000, scales=0x2000000, biases=0x3000000, y=0x10000 + 64, n=64)]), "operand"),
    (dict(segs=[dict(w=0x1000000, scales=0x2000000, biases=0x3000000, y=0x1000000 + 64, n=64)]), "weight"),
    (dict(n_segs=2, segs=[dict(w=0x1000000, scales=0x2000000, biases=0x3000000, y=0x4000000, n=64),
                          dict(w=0x5000000, scales=0x6000000, biases=0x7000000, y=0x4000000 + 2, n=8)]),
     "overlap"),
])
def test_qlinear_rejects_bad_arguments(gdn, kw, msg):
    rc = gdn.lib().gdn_qlinear(ctypes.byref(_ql(gdn, **kw)))
    assert rc == gdn.GDN_EINVAL
    assert msg in gdn.last_error(), gdn.last_error()


def test_qlinear_workspace_size(gdn):
    """GEMV path (m <= 4 and m k <= 30720): none. MFMA path: the operand in fragment order,
    1 KB per (16-row tile, 32 values), the tile count rounded up to the tiles a workgroup
    takes (up to 4), then the operand's fp32 sum per (row, 64 values); both 256-byte
    aligned."""
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731

    def ws(tiles, k, layers=1):
        return al(layers * tiles * (k // 32) * 1024) + al(layers * 16 * tiles * (k // 64) * 4)
    assert gdn.qlinear_workspace_size(4, 5120) == 0
    assert gdn.qlinear_workspace_size(1, 8192) == 0
    assert gdn.qlinear_workspace_size(4, 8192) == ws(1, 8192)
    assert gdn.qlinear_workspace_size(5, 5120) == ws(1, 5120)
    assert gdn.qlinear_workspace_size(40, 5120) == ws(3, 5120) == 3 * 160 * 1024 + 3 * 16 * 80 * 4
    assert gdn.qlinear_workspace_size(40, 6144, n_layers=2) == ws(3, 6144, 2)
    assert gdn.qlinear_workspace_size(65, 5120) == ws(8, 5120)  # 5 tiles -> 2 x 4
    assert gdn.qlinear_workspace_size(512, 1024) == ws(32, 1024)
    assert gdn.qlinear_workspace_size(1024, 5120) == ws(64, 5120)
    assert gdn.qlinear_workspace_size(4096, 8192) == ws(256, 8192)
    with pytest.raises(gdn.GdnError):
        gdn.qlinear_workspace_size(4097, 5120)


@pytest.mark.parametrize("kw,msg", [
    (dict(m=40, workspace=0x8000000, workspace_bytes=1 << 30), "takes no workspace"),
    (dict(m=4, workspace_bytes=16), "takes no workspace"),
    (dict(n_layers=2, m=512, k=8192), "more than the 9437184"),
    (dict(n_layers=48, m=40, k=5120), "more than the 9437184"),
    (dict(m=1024, k=8192), "more than the 9437184"),
    (dict(m=4097), "bad shape"),
    (dict(x=None), "exactly one"),
])
def test_qlinear_noalloc_rejects_bad_arguments(gdn, kw, msg):
    """The no-allocation variant takes no workspace and refuses shapes whose operand does not
    fit the library's scratch (GDN_QLINEAR_NOALLOC_SCRATCH_BYTES); its other checks are
    gdn_qlinear's."""
    rc = gdn.lib().gdn_qlinear_noalloc(ctypes.byref(_ql(gdn, **kw)))
    assert rc == gdn.GDN_EINVAL
    assert msg in gdn.last_error(), gdn.last_error()
    assert gdn.last_error().startswith("gdn_qlinear_noalloc:")


def test_qlinear_noalloc_scratch_fits_one_layer(gdn):
    """One layer at 512 rows and the largest k (8 MiB of operand, 256 KiB of group sums)
    fits the scratch, as do 1024 rows up to k = 4096; two layers at 512 rows do not."""
    assert gdn.qlinear_workspace_size(512, 8192) == (8 << 20) + (256 << 10)
    assert gdn.qlinear_workspace_size(512, 8192) <= gdn.QLINEAR_NOALLOC_SCRATCH_BYTES
    assert gdn.qlinear_workspace_size(1024, 4096) <= gdn.QLINEAR_NOALLOC_SCRATCH_BYTES
    assert gdn.qlinear_workspace_size(512, 8192, n_layers=2) > gdn.QLINEAR_NOALLOC_SCRATCH_BYTES
    text = open(HEADER).read()
    assert "#define GDN_QLINEAR_NOALLOC_SCRATCH_BYTES ((size_t)9 << 20)" in text


def test_length_dispatch_follows_the_measured_crossover(gdn):
    """A non-recording call runs the chunked form from the measured crossover on (about 36,
    32, 30, 32 tokens for 1, 2, 4, 8 sequences; 32 from 5 on), shorter ones and recording
    ones the recurrent kernel (python/qwen35.py:606-626 chooses by length the same way)."""
    import torch
    x = torch.zeros(64, dtype=torch.bfloat16)  # 16-byte aligned host buffer: the choice only reads its address
    use = gdn.gdn._use_chunked
    for B, first in ((1, 36), (2, 32), (3, 31), (4, 30), (5, 32), (8, 32), (64, 32)):
        assert gdn.chunked_min_t(B) == first
        assert not use(B, first - 1, False, x, None, (x,))
        assert use(B, first, False, x, None, (x,))
        assert not use(B, 4096, True, x, None, (x,))
