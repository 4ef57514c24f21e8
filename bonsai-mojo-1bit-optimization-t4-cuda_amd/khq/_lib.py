"""ctypes binding of libkhq_hip.so (the C ABI declared in include/khq.h).

This mirrors how the reference binds its native library
(ref:src/ops.mojo:585-611, 1101-1279): the shared object is opened once and
each launcher is called with raw device pointers and plain ints/floats.  The
wrappers below take torch tensors (or raw ints) and pass the current HIP
stream.  There is no fallback: if the library is missing or a launch fails,
an exception is raised.
"""
from __future__ import annotations

import ctypes
import os

from .build import LIB_PATH

_lib = None

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float

# name -> argtypes (all return int)
SIGNATURES = {
    "launch_khq_compress_fp16": [P] * 10 + [I, I, F, F, I, P],
    "launch_khq_attn_fp16": [P] * 18 + [I, I, I, I, I, I, F, F, F, F, I, I, P],
    "launch_khq_window_attn_fp16": [P] * 4 + [I, I, I, I, I, I, F, P],
    "launch_khq_gather_q_fp16": [P, P, I, I, P],
    "launch_khq_merge_gate_fp16": [P, P, P, P, I, I, I, P],
    "launch_khq_ring_write_fp16": [P] * 6 + [I, I, P],
    "launch_khq_partial_rope_fp16": [P, I, I, I, I, F, I, P],
    "launch_khq_gqa_attn_fp16": [P] * 4 + [I, I, I, I, F, P],
    "khq_attn_step_fp16": [P] * 19 + [I, I, I, I, I, I, F, F, F, F, P],
    "khq_attn_step_noalloc_fp16": [P] * 19 + [I, I, I, I, I, I, F, F, F, F, P],
    "khq_attn_step_batched_fp16": [P, I] + [P] * 7 + [I, I, F, F, F, F, P],
    "khq_decompress_fp16": [P] * 15 + [I, I, I, I, F, F, F, P, I, P, I, P],
    "khq_prefill_attn_fp16": [P, P, P, I, I, I, I, I, I, F, P, P],
    "khq_prefill_attn_partials_fp16": [P, P, P, I, I, I, I, I, I, F, P],
    "khq_attn_partials_fp16": [P] * 16 + [I, I, I, F, F, F, F, P],
    "khq_attn_parts": [I],
    "khq_select_kernel": [I],
    "khq_workspace_reserve": [ctypes.c_size_t],
    "khq_attn_reduce_f32": [P, P, I, I, P],
    "khq_fault_status": [P, I],
    "khq_set_spin_limit": [I],
    # per-layer runtime
    "khq_layer_create": [I, I, I] + [P] * 7 + [F, F, F, F, F, I, I],
    "khq_layer_destroy": [P],
    "khq_layer_reset": [P],
    "khq_layer_state": [P, P, P, P],
    "khq_layer_payload": [P, P],
    "khq_layer_dense": [P, P, P, P, P],
    "khq_layer_capture_unroped": [P, P, P],
    "khq_layer_step": [P] * 6 + [F, P],
    "khq_layer_prefill": [P] * 6 + [I, F, P],
    # calibration dumps
    "khq_dump_create": [ctypes.c_char_p, I, I, I],
    "khq_dump_destroy": [P],
    "khq_dump_count": [P, I],
    "khq_dump_kv": [P, I, P, P, P],
    "khq_dump_attn": [P, I, P, P, I, I, I, I, F, P],
    "khq_dump_flush": [P],
    "khq_layer_set_dump": [P, P, I],
    # calibration
    "launch_cal_op": [I] + [P] * 7 + [F, F, I, I, I, I, P],
    "launch_cal_svq_train": [P] * 6 + [I, I, I, I, I, I, F, P],
    "launch_cal_svq_pass": [P] * 8 + [I, I, I, I, F, P],
    "khq_layer_attention_step": [P] * 6 + [F, I, P, F, P],
}
# return types other than int
RESTYPES = {"khq_layer_create": ctypes.c_void_p, "khq_layer_destroy": None,
            "khq_dump_create": ctypes.c_void_p, "khq_dump_destroy": None}


class KhqSeq(ctypes.Structure):
    """struct khq_seq of include/khq.h: one sequence of a batched step."""

    _fields_ = [(n, P) for n in ("q_gate", "k_payload", "v_payload", "v_shared_meta", "k_mask",
                                 "k_norms", "k_r_norms", "v_norms", "v_r_norms", "ring_k",
                                 "ring_v", "out")] + [
        (n, I) for n in ("c_len", "win_start", "win_len", "ring_cap")]


class KhqError(RuntimeError):
    """A launcher returned a nonzero code (-100 bad shape, -101 missing
    split buffer, > 0 a hipError_t)."""

    def __init__(self, name: str, rc: int):
        super().__init__(f"{name} returned {rc}")
        self.rc = rc


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
        _lib = ctypes.CDLL(LIB_PATH, mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        _lib.khq_version.restype = ctypes.c_char_p
    return _lib


def ptr(t) -> int | None:
    """Device pointer of a tensor (or None / raw int passthrough)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def stream_handle(stream=None) -> int | None:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream or None


def call(name: str, *args, check: bool = True) -> int:
    rc = getattr(lib(), name)(*args)
    if check and rc != 0:
        raise KhqError(name, rc)
    return rc


def version() -> str:
    return lib().khq_version().decode()
