"""ctypes front end of the CPU oracle (oracle/khq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the product.

Every entry point mirrors one C-ABI launcher of the HIP library (same argument
order and error codes) but takes numpy arrays.  fp16 data is passed as
numpy.float16 arrays (bit-identical to uint16 storage).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkhq_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile oracle/libkhq_oracle.so with oracle/Makefile."""
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.khq_h2f.restype = ctypes.c_float
        _lib.khq_h2f.argtypes = [ctypes.c_uint16]
        _lib.khq_f2h.restype = ctypes.c_uint16
        _lib.khq_f2h.argtypes = [ctypes.c_float]
        _lib.khq_ref_num_threads.restype = ctypes.c_int
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def num_threads() -> int:
    return int(lib().khq_ref_num_threads())


def set_num_threads(n: int) -> None:
    lib().khq_ref_set_num_threads(ctypes.c_int(n))


def f2h(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.float16)
    lib().khq_f2h_array(_p(a), _p(out), ctypes.c_long(a.size))
    return out


def compress(x, d_vec, rotor, cents, vq, ts: float, alpha: float, is_v: bool):
    """Restates launch_khq_compress_fp16 (ref .cu:4279-4310) on host arrays.

    Returns (rc, mask[n,16] u32, norms[n] f16, r_norms[n] f16,
    payload[n,40|104] u8, shared_meta[n,4] u8)."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    n = x.shape[0] if x.ndim == 2 else 0
    d = x.shape[1] if x.ndim == 2 else 0
    stride = 104 if is_v else 40
    mask = np.zeros((max(n, 1), 16), np.uint32)
    norms = np.zeros(max(n, 1), np.float16)
    rn = np.zeros(max(n, 1), np.float16)
    pay = np.zeros((max(n, 1), stride), np.uint8)
    sm = np.zeros((max(n, 1), 4), np.uint8)
    args = [np.ascontiguousarray(a, dtype=np.float16) for a in (d_vec, rotor, cents, vq)]
    rc = lib().khq_ref_compress(
        _p(x), *[_p(a) for a in args], _p(mask), _p(norms), _p(rn), _p(pay), _p(sm),
        ctypes.c_int(n), ctypes.c_int(d), ctypes.c_float(ts), ctypes.c_float(alpha),
        ctypes.c_int(1 if is_v else 0))
    return rc, mask[:n], norms[:n], rn[:n], pay[:n], sm[:n]


def attn(q_gate, kpay, vpay, vsm, kmask, knorm, krn, vnorm, vrn, cents_k, cents_v,
         vq, rotor_k, rotor_v, dk, dv, *, num_queries, num_heads, L_q, c_len,
         n_rep, scale, alpha_k, alpha_v, rope_base, start_pos, num_splits,
         stride_s=0, with_partial=True):
    """Restates launch_khq_attn_fp16 (ref .cu:4314-4375).

    Returns (rc, out_attn[num_queries, 258] f32, out_partial or None)."""
    out = np.zeros((num_queries if num_queries > 0 else 1, 258), np.float32)
    ns = max(num_splits, 1)
    part = np.zeros((max(num_queries, 1), ns, 258), np.float32) if with_partial else None
    h16 = [np.ascontiguousarray(a, dtype=np.float16)
           for a in (q_gate, knorm, krn, vnorm, vrn, cents_k, cents_v, vq, rotor_k, rotor_v, dk, dv)]
    qg, knorm, krn, vnorm, vrn, cents_k, cents_v, vq, rotor_k, rotor_v, dk, dv = h16
    kpay = np.ascontiguousarray(kpay, dtype=np.uint8)
    vpay = np.ascontiguousarray(vpay, dtype=np.uint8)
    vsm = np.ascontiguousarray(vsm, dtype=np.uint8)
    kmask = np.ascontiguousarray(kmask, dtype=np.uint32)
    rc = lib().khq_ref_attn(
        _p(qg), _p(kpay), _p(vpay), _p(vsm), _p(kmask), _p(knorm), _p(krn), _p(vnorm),
        _p(vrn), _p(cents_k), _p(cents_v), _p(vq), _p(rotor_k), _p(rotor_v), _p(dk), _p(dv),
        _p(out), _p(part), ctypes.c_int(num_queries), ctypes.c_int(num_heads),
        ctypes.c_int(L_q), ctypes.c_int(c_len), ctypes.c_int(stride_s), ctypes.c_int(n_rep),
        ctypes.c_float(scale), ctypes.c_float(alpha_k), ctypes.c_float(alpha_v),
        ctypes.c_float(rope_base), ctypes.c_int(start_pos), ctypes.c_int(num_splits))
    return rc, out, part


def window_attn(q_gate, ring_k, ring_v, *, win_start, win_len, ring_cap, H_q, H_kv,
                d=256, scale):
    """Restates launch_khq_window_attn_fp16 (ref .cu:4378-4396)."""
    out = np.zeros((max(H_q, 1), d + 2), np.float32)
    qg = np.ascontiguousarray(q_gate, dtype=np.float16)
    rk = np.ascontiguousarray(ring_k, dtype=np.float16)
    rv = np.ascontiguousarray(ring_v, dtype=np.float16)
    rc = lib().khq_ref_window_attn(
        _p(qg), _p(rk), _p(rv), _p(out), ctypes.c_int(win_start), ctypes.c_int(win_len),
        ctypes.c_int(ring_cap), ctypes.c_int(H_q), ctypes.c_int(H_kv), ctypes.c_int(d),
        ctypes.c_float(scale))
    return rc, out


def merge_gate(attn_c, attn_w, q_gate, *, H_q, d=256, has_w):
    """Restates launch_khq_merge_gate_fp16 (ref .cu:4414-4429)."""
    out = np.zeros((max(H_q, 1), d), np.float16)
    ac = np.ascontiguousarray(attn_c, dtype=np.float32)
    aw = np.ascontiguousarray(attn_w if attn_w is not None else attn_c, dtype=np.float32)
    qg = np.ascontiguousarray(q_gate, dtype=np.float16)
    rc = lib().khq_ref_merge_gate(_p(ac), _p(aw), _p(qg), _p(out), ctypes.c_int(H_q),
                                  ctypes.c_int(d), ctypes.c_int(1 if has_w else 0))
    return rc, out


def gather_q(q_gate, *, H_q, d=256):
    out = np.zeros((max(H_q, 1), d), np.float16)
    qg = np.ascontiguousarray(q_gate, dtype=np.float16)
    rc = lib().khq_ref_gather_q(_p(qg), _p(out), ctypes.c_int(H_q), ctypes.c_int(d))
    return rc, out


def partial_rope_fp16(vec, *, num_heads, head_dim, rotary_dim, pos, theta, stride=0):
    """Restates partial_rope_sm75_gpu (ref elementwise_sm75.mojo:1023-1061) in place."""
    v = np.ascontiguousarray(vec, dtype=np.float16).copy()
    lib().khq_ref_partial_rope_fp16(_p(v), ctypes.c_int(num_heads), ctypes.c_int(head_dim),
                                    ctypes.c_int(rotary_dim), ctypes.c_int(pos),
                                    ctypes.c_float(theta), ctypes.c_int(stride))
    return v


def gqa_host(q_gate, k_cache, v_cache, *, seq_len, H_q, H_kv, D=256, scale):
    """Restates the fp32 host attention of ref attention.mojo:175-196."""
    out = np.zeros((H_q, D), np.float32)
    qg = np.ascontiguousarray(q_gate, dtype=np.float16)
    kc = np.ascontiguousarray(k_cache, dtype=np.float16)
    vc = np.ascontiguousarray(v_cache, dtype=np.float16)
    lib().khq_ref_gqa_host(_p(qg), _p(kc), _p(vc), _p(out), ctypes.c_int(seq_len),
                           ctypes.c_int(H_q), ctypes.c_int(H_kv), ctypes.c_int(D),
                           ctypes.c_float(scale))
    return out
