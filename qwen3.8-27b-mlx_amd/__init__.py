"""MI355X-native (gfx950) gated-delta recurrence: HIP kernels behind the C ABI of
include/gdn.h, with a Python mirror of the reference's per-layer interface."""
from .gdn import (  # noqa: F401
    CHUNKED_MIN_T, chunked_min_t, CONV_TAPS, DTYPE_BF16, DTYPE_F32, EXPORTS, FRONTEND_CONV, FRONTEND_QKV, GATES_PRECOMPUTED,
    GATES_RAW, GDN_EDEVICE, GDN_EINVAL, GDN_EUNSUPPORTED, GDN_OK, HEAD_DIM, LIB_PATH, PREFILL_FAST, PREFILL_ACCURATE,
    STATES_BHT, STATES_TBH, CommitArgs, DeltaCache, GdnError, LayerArgs, Result, available,
    call_commit, call_prefill, call_prefill_timed, call_qlinear, call_qlinear_noalloc, call_run, commit, last_error, layer, layer_args,
    lib, prefill_chunked, prefill_workspace_size, qlinear, qlinear_args, QLinearArgs,
    QLinearSeg, QuantLinear, QLINEAR_GEMV_ROWS, QLINEAR_MAX_ROWS, QLINEAR_MAX_SEGS,
    QLINEAR_NOALLOC_SCRATCH_BYTES, qlinear_noalloc, qlinear_workspace_size, run,
)
from . import weights  # noqa: F401,E402  (checkpoint reader for the path's weights)
