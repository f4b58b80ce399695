"""ctypes binding of libdspine_verify.so (the C ABI declared in include/dspine_verify.h).

The library is built in-tree by ``dspine_amd/csrc/build.py`` (``__graft_entry__.build()``).
There is no fallback: every product entry point raises when the library is missing.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdspine_verify.so")

DSV_OK, DSV_ERR_INVALID, DSV_ERR_UNSUPPORTED, DSV_ERR_LAUNCH, DSV_ERR_WORKSPACE = range(5)
DSV_F32, DSV_BF16, DSV_F16 = 0, 1, 2
DSV_BACKEND_PYTORCH, DSV_BACKEND_FLASHINFER = 0, 1
LIST_K = 64

# Every symbol include/dspine_verify.h declares (checked by tests/test_lib_symbols.py).
EXPORTS = (
    "dsv_last_error", "dsv_device_count", "dsv_verify_workspace_bytes", "dsv_verify",
    "dsv_greedy_verify", "dsv_greedy_workspace_bytes", "dsv_topk", "dsv_topk_workspace_bytes",
    "dsv_uniforms", "dsv_profile_events", "dsv_adjust_logits", "dsv_adjust_history",
    "dsv_logits_padding", "dsv_window_index", "dsv_target_probs", "dsv_compress",
    "dsv_accept_chain", "dsv_sample_chain", "dsv_pack_joint", "dsv_sps_plan",
    "dsv_greedy_verify_noalloc", "dsv_commit_accept", "dsv_rs_table", "dsv_rs_table_workspace_bytes",
    "dsv_factor_table", "dsv_factor_direct", "dsv_factor_workspace_doubles", "dsv_factor_widen",
    "dsv_factor_gemm", "dsv_filter_probs", "dsv_filter_workspace_bytes",
)
DSV_ADJ_ADD, DSV_ADJ_SCALE = 0, 1

_c = ctypes
vp, i32, i64 = _c.c_void_p, _c.c_int32, _c.c_int64


class VerifyArgs(ctypes.Structure):
    """Mirror of ``dsv_verify_args``."""

    _fields_ = [
        ("logits", vp), ("logits_dtype", i32), ("stages", i32),
        ("rows", i64), ("vocab", i64), ("row_stride", i64),
        ("bs", i32), ("T", i32),
        ("verify_lens", vp), ("row_offsets", vp), ("row_offsets_i64", i32),
        ("backend", i32),
        ("temperatures", vp), ("top_ks", vp), ("top_ps", vp), ("min_ps", vp),
        ("filter", i32), ("need_min_p", i32), ("any_greedy", i32), ("max_top_k", i32),
        ("sparse_joint", i32), ("pad0", i32),
        ("hist_ids", vp), ("hist_len", i32), ("pad1", i32), ("presence", vp), ("repetition", vp),
        ("candidates", vp), ("q_ids", vp), ("q_ids_i64", i32), ("K", i32), ("q_values", vp),
        ("uniforms", vp), ("uniform_final", vp), ("prefix_lens", vp),
        ("page_table", vp), ("page_stride", i64), ("page_cols", i64),
        ("accept", vp), ("commit", vp), ("bonus", vp), ("output", vp), ("new_seq", vp),
        ("kv_slots", vp),
        ("workspace", vp), ("workspace_bytes", i64),
    ]


class ChainArgs(ctypes.Structure):
    """Mirror of ``dsv_chain_args``."""

    _fields_ = [
        ("bs", i32), ("T", i32), ("K", i32), ("pad0", i32),
        ("vocab", i64),
        ("candidates", vp), ("verify_lens", vp), ("uniforms", vp), ("uniform_final", vp),
        ("prefix_lens", vp),
        ("row_offsets", vp), ("row_offsets_i64", i32), ("pad1", i32),
        ("dense_p", vp), ("p_stride", i64), ("denominator", vp),
        ("p_ids", vp), ("p_values", vp), ("p_lengths", vp), ("p_overflow", vp),
        ("p_cap", i32), ("pad2", i32),
        ("dense_q", vp), ("q_stride", i64),
        ("q_ids", vp), ("q_ids_i64", i32), ("pad3", i32), ("q_values", vp),
        ("accept", vp), ("commit", vp), ("bonus", vp), ("output", vp), ("new_seq", vp),
        ("overflow_read", vp),
    ]


class FactorArgs(ctypes.Structure):
    """Mirror of ``dsv_factor_args``."""

    _fields_ = [
        ("n", i64), ("K", i32), ("T", i32), ("H", i32), ("R", i32), ("vocab", i64),
        ("raw", vp), ("raw_dtype", i32), ("query_dtype", i32), ("raw_stride", i64),
        ("rms", vp), ("query", vp), ("query_stride", i64), ("anchors", vp), ("cand", vp),
        ("W", vp), ("gram", vp), ("G", vp), ("Vm", vp), ("TG", vp), ("bias", vp), ("norm", vp),
        ("head", vp), ("candidate_head", vp), ("head_dtype", i32), ("pad0", i32), ("head_stride", i64),
        ("eps", _c.c_double), ("out", vp), ("base_out", vp), ("x", vp), ("scale", vp), ("first", vp),
        ("message", vp), ("tg", vp), ("safe", vp), ("d", vp), ("magnitude", vp), ("y", vp),
        ("gemm_ws", vp), ("gemm_ws_doubles", i64),
    ]


_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
    pass


def load():
    """Load (once) the HIP library; raise when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        lib = ctypes.CDLL(LIB_PATH)
        lib.dsv_last_error.restype = ctypes.c_char_p
        lib.dsv_device_count.restype = i32
        lib.dsv_verify_workspace_bytes.restype = i64
        lib.dsv_verify_workspace_bytes.argtypes = [i64, i32, i32, i64]
        lib.dsv_greedy_workspace_bytes.restype = i64
        lib.dsv_greedy_workspace_bytes.argtypes = [i64, i64]
        lib.dsv_topk_workspace_bytes.restype = i64
        lib.dsv_topk_workspace_bytes.argtypes = [i64, i64, i32]
        lib.dsv_verify.restype = i32
        lib.dsv_verify.argtypes = [ctypes.POINTER(VerifyArgs), vp]
        lib.dsv_greedy_verify.restype = i32
        lib.dsv_greedy_verify.argtypes = [vp, i32, i64, i64, i64, i32, i32, vp, vp, i32, vp,
                                          vp, vp, vp, vp, vp, vp, vp, i64, vp]
        lib.dsv_greedy_verify_noalloc.restype = i32
        lib.dsv_greedy_verify_noalloc.argtypes = [vp, i32, i64, i64, i64, i32, i32, vp, vp, i32, vp,
                                                  vp, vp, vp, vp, vp, vp, vp]
        lib.dsv_topk.restype = i32
        lib.dsv_topk.argtypes = [vp, i32, i64, i64, i64, i32, vp, vp, i32, vp, i64, vp]
        lib.dsv_uniforms.restype = i32
        lib.dsv_uniforms.argtypes = [vp, vp, i32, i64, i32, i32, vp, vp]
        lib.dsv_profile_events.restype = i32
        lib.dsv_profile_events.argtypes = [vp, vp]
        lib.dsv_adjust_logits.restype = i32
        lib.dsv_adjust_logits.argtypes = [vp, i32, i64, i64, i64, vp, i32, i64, i32, vp, i64, vp]
        lib.dsv_adjust_history.restype = i32
        lib.dsv_adjust_history.argtypes = [vp, i32, i64, i64, i64, vp, i32, i64, vp, i32, vp, vp, vp]
        lib.dsv_logits_padding.restype = i32
        lib.dsv_logits_padding.argtypes = [vp, i32, i64, i64, i64, vp]
        lib.dsv_window_index.restype = i32
        lib.dsv_window_index.argtypes = [vp, i32, i32, i32, vp, i64, vp]
        lib.dsv_target_probs.restype = i32
        lib.dsv_target_probs.argtypes = [ctypes.POINTER(VerifyArgs), vp, i64, i32, vp]
        lib.dsv_filter_probs.restype = i32
        lib.dsv_filter_probs.argtypes = [ctypes.POINTER(VerifyArgs), vp, i64, vp, i64, i32, i32, vp]
        lib.dsv_filter_workspace_bytes.restype = i64
        lib.dsv_filter_workspace_bytes.argtypes = [i64, i64]
        lib.dsv_compress.restype = i32
        lib.dsv_compress.argtypes = [vp, i64, i64, i64, i32, vp, vp, vp, vp, vp]
        lib.dsv_accept_chain.restype = i32
        lib.dsv_accept_chain.argtypes = [ctypes.POINTER(ChainArgs), vp]
        lib.dsv_pack_joint.restype = i32
        lib.dsv_pack_joint.argtypes = [vp, vp, i64, i32, vp, vp, i32, vp, vp, vp, vp, vp, i64, i64, vp]
        lib.dsv_sample_chain.restype = i32
        lib.dsv_sample_chain.argtypes = [vp, i64, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.dsv_rs_table_workspace_bytes.restype = i64
        lib.dsv_rs_table_workspace_bytes.argtypes = [i64, i32, i32, i32]
        lib.dsv_rs_table.restype = i32
        lib.dsv_rs_table.argtypes = [vp, i64, vp, vp, i64, vp, vp, i64, i32, i32, vp, i32, vp, vp, vp, vp, i32, i32,
                                     vp, vp, i32, vp, vp, i32, _c.c_float, vp, vp, i64, vp]
        lib.dsv_commit_accept.restype = i32
        lib.dsv_commit_accept.argtypes = [i32, i32, vp, vp, vp, i32, vp, i32, vp, i64, i64, vp, vp, vp, i32, vp, vp,
                                          vp]
        lib.dsv_factor_workspace_doubles.restype = i64
        lib.dsv_factor_workspace_doubles.argtypes = [i64, i32, i32, i32]
        lib.dsv_factor_table.restype = i32
        lib.dsv_factor_table.argtypes = [ctypes.POINTER(FactorArgs), vp]
        lib.dsv_factor_direct.restype = i32
        lib.dsv_factor_direct.argtypes = [ctypes.POINTER(FactorArgs), vp]
        lib.dsv_factor_widen.restype = i32
        lib.dsv_factor_widen.argtypes = [vp, i32, i64, i64, i64, _c.c_double, vp, vp, vp]
        lib.dsv_factor_gemm.restype = i32
        lib.dsv_factor_gemm.argtypes = [vp, i64, i64, vp, i64, i64, vp, i64, i64, i64, i32, vp]
        lib.dsv_sps_plan.restype = i32
        lib.dsv_sps_plan.argtypes = [vp, i64, i32, i32, vp, i64, i32, i64, vp, vp, i32, i32, vp, vp, vp, vp]
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Map a library status onto the reference's exception types (ValueError for contract
    violations before launch, RuntimeError for launch failures)."""
    if rc == DSV_OK:
        return
    msg = load().dsv_last_error().decode(errors="replace")
    if rc in (DSV_ERR_INVALID, DSV_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    if rc == DSV_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return DSV_BF16
    if t.dtype == torch.float32:
        return DSV_F32
    raise ValueError(f"unsupported logits dtype {t.dtype} (expected float32 or bfloat16)")


def require_cuda(*tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("the HIP verification path requires device (cuda) tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on one device")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev
