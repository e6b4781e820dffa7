"""ctypes binding of ``libtreeattn_amd.so`` (declared in ``include/treeattn_amd.h``).

The library is built in-tree by ``treeattention_amd/build.py``.  There is no
CPU or Python fallback: every entry point raises when the library is missing.
"""

from __future__ import annotations

import ctypes
import os
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libtreeattn_amd.so")

TA_OK = 0
TA_ERR_INVALID, TA_ERR_UNSUPPORTED, TA_ERR_LAUNCH = 1, 2, 3
TA_F32, TA_BF16, TA_F16 = 0, 1, 2
TA_TREE_NATURAL, TA_TREE_COMPAT, TA_TREE_NODEKEYS = 0, 1, 2
TA_CAUSAL_NONE, TA_CAUSAL_EXACT, TA_CAUSAL_REFERENCE = 0, 1, 2

TREE_MODES = {"natural": TA_TREE_NATURAL, "compat": TA_TREE_COMPAT, "nodekeys": TA_TREE_NODEKEYS}

_I64x3 = ctypes.c_int64 * 3


class Problem(ctypes.Structure):
    """Mirror of ``ta_problem``."""

    _fields_ = [
        ("B", ctypes.c_int64),
        ("L", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("num_samples", ctypes.c_int64),
        ("branching", ctypes.c_int64),
        ("leaf_block", ctypes.c_int64),
        ("tree_mode", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("dense_cols", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("max_logit", ctypes.c_float),
        ("q_strides", _I64x3),
        ("k_strides", _I64x3),
        ("v_strides", _I64x3),
        ("o_strides", _I64x3),
        ("g_strides", _I64x3),
        ("w_strides", _I64x3),
    ]


EXPORTS = (
    "ta_version",
    "ta_last_error",
    "ta_record_bytes",
    "ta_forward_workspace_bytes",
    "ta_backward_workspace_bytes",
    "ta_record_offset",
    "ta_fill_uniforms",
    "ta_pool",
    "ta_sample",
    "ta_bucket",
    "ta_leaf_forward",
    "ta_forward",
    "ta_leaf_backward",
    "ta_tree_backward",
    "ta_backward",
    "ta_det_weights",
    "ta_det_grad",
    "ta_haar_workspace_bytes",
    "ta_haar_keys",
    "ta_haar_keys_adjoint",
    "ta_det_stream_forward",
    "ta_det_stream_backward",
    "ta_path_bytes",
    "ta_pack_paths",
    "ta_unpack_paths",
    "ta_replay",
    "ta_forward_replay",
    "ta_forward_static",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _declare(lib: ctypes.CDLL) -> None:
    P = ctypes.POINTER(Problem)
    vp = ctypes.c_void_p
    i64p = ctypes.POINTER(ctypes.c_int64)
    lib.ta_version.restype = ctypes.c_int
    lib.ta_version.argtypes = []
    lib.ta_last_error.restype = ctypes.c_char_p
    lib.ta_last_error.argtypes = []
    for name in ("ta_record_bytes", "ta_forward_workspace_bytes", "ta_backward_workspace_bytes"):
        f = getattr(lib, name)
        f.restype = ctypes.c_int
        f.argtypes = [P, i64p]
    lib.ta_record_offset.restype = ctypes.c_int
    lib.ta_record_offset.argtypes = [P, ctypes.c_int, i64p]
    lib.ta_fill_uniforms.restype = ctypes.c_int
    lib.ta_fill_uniforms.argtypes = [ctypes.c_uint64, ctypes.c_int64, vp, vp]
    lib.ta_pool.restype = ctypes.c_int
    lib.ta_pool.argtypes = [P, vp, vp, vp]
    lib.ta_sample.restype = ctypes.c_int
    lib.ta_sample.argtypes = [P, vp, vp, ctypes.c_uint64, vp, vp, vp]
    lib.ta_bucket.restype = ctypes.c_int
    lib.ta_bucket.argtypes = [P, vp, vp]
    lib.ta_leaf_backward.restype = ctypes.c_int
    lib.ta_leaf_backward.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ta_tree_backward.restype = ctypes.c_int
    lib.ta_tree_backward.argtypes = [P, vp, vp, vp, vp, vp, vp, vp]
    lib.ta_leaf_forward.restype = ctypes.c_int
    lib.ta_leaf_forward.argtypes = [P, vp, vp, vp, vp, vp, vp, vp]
    lib.ta_forward.restype = ctypes.c_int
    lib.ta_forward.argtypes = [P, vp, vp, vp, vp, ctypes.c_uint64, vp, vp, vp, vp, vp]
    lib.ta_backward.restype = ctypes.c_int
    lib.ta_backward.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    i64 = ctypes.c_int64
    lib.ta_det_weights.restype = ctypes.c_int
    lib.ta_det_weights.argtypes = [vp, i64, vp, i64, i64, i64, i64, ctypes.c_int, vp]
    lib.ta_det_grad.restype = ctypes.c_int
    lib.ta_det_grad.argtypes = [vp, i64, vp, vp, i64, i64, i64, ctypes.c_int, vp]
    lib.ta_haar_keys.restype = ctypes.c_int
    lib.ta_haar_keys.argtypes = [ctypes.c_int, vp, i64p, vp, vp, i64, i64, i64, i64, vp]
    lib.ta_haar_workspace_bytes.restype = ctypes.c_int
    lib.ta_haar_workspace_bytes.argtypes = [i64, i64, i64, i64, i64p]
    lib.ta_haar_keys_adjoint.restype = ctypes.c_int
    lib.ta_haar_keys_adjoint.argtypes = [ctypes.c_int, vp, vp, i64p, i64, i64, i64, i64, vp]
    lib.ta_det_stream_forward.restype = ctypes.c_int
    lib.ta_det_stream_forward.argtypes = [ctypes.c_int, vp, i64p, vp, i64p, vp, i64p, vp, i64p, vp, i64, i64, i64,
                                          i64, i64, ctypes.c_int, vp]
    lib.ta_det_stream_backward.restype = ctypes.c_int
    lib.ta_det_stream_backward.argtypes = [ctypes.c_int, vp, i64p, vp, i64p, vp, i64p, vp, i64p, vp, vp, vp, vp, vp,
                                           vp, i64p, i64, i64, i64, i64, i64, ctypes.c_int, vp]
    lib.ta_path_bytes.restype = ctypes.c_int
    lib.ta_path_bytes.argtypes = [i64, i64p]
    lib.ta_pack_paths.restype = ctypes.c_int
    lib.ta_pack_paths.argtypes = [vp, i64p, i64, i64, i64, i64, i64, vp, vp]
    lib.ta_unpack_paths.restype = ctypes.c_int
    lib.ta_unpack_paths.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64p, vp]
    lib.ta_replay.restype = ctypes.c_int
    lib.ta_replay.argtypes = [P, vp, vp, vp, vp, vp]
    lib.ta_forward_replay.restype = ctypes.c_int
    lib.ta_forward_replay.argtypes = [P, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ta_forward_static.restype = ctypes.c_int
    lib.ta_forward_static.argtypes = [P, vp, vp, vp, vp, ctypes.c_uint64, vp, vp, vp, vp]


def load() -> ctypes.CDLL:
    """Loads the library (once); raises ``RuntimeError`` if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"tree-attention HIP library not found at {LIB_PATH}; "
                    "build it with `python -m treeattention_amd.build` (hipcc, gfx950)"
                )
            lib = ctypes.CDLL(LIB_PATH)
            _declare(lib)
            if lib.ta_version() != 1:
                raise RuntimeError(f"unexpected library version {lib.ta_version()}")
            _lib = lib
    return _lib


def check(rc: int) -> None:
    """Raises ``RuntimeError`` with the library's message for a non-zero code."""
    if rc != TA_OK:
        msg = load().ta_last_error().decode(errors="replace")
        if rc in (1, 2):
            raise ValueError(msg) if rc == 1 else NotImplementedError(msg)
        raise RuntimeError(msg)


TA_REC_LEAVES, TA_REC_SUMMARIES, TA_REC_NUM_ROWS = 0, 1, 2


def record_offset(prob: Problem, which: int) -> int:
    out = ctypes.c_int64()
    check(load().ta_record_offset(ctypes.byref(prob), which, ctypes.byref(out)))
    return out.value


def byte_sizes(prob: Problem) -> tuple[int, int, int]:
    """(record, forward workspace, backward workspace) bytes for ``prob``."""
    lib = load()
    r, f, b = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    check(lib.ta_record_bytes(ctypes.byref(prob), ctypes.byref(r)))
    check(lib.ta_forward_workspace_bytes(ctypes.byref(prob), ctypes.byref(f)))
    check(lib.ta_backward_workspace_bytes(ctypes.byref(prob), ctypes.byref(b)))
    return r.value, f.value, b.value
