"""Torch-tensor front end of the C ABI (one function per launcher).

Each function checks tensor shapes/dtypes/devices on the host before the
launch (a kernel must never see a shape its grid does not assume), then calls
the launcher through ctypes on the current HIP stream.  Names and argument
meaning follow the reference's FFI wrappers (ref:src/ops.mojo:1101-1279).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import call, ptr, stream_handle

D = 256
ROW_BYTES = 220


def _need(t: torch.Tensor, dtype, numel: int | None = None, name: str = "tensor"):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements, need >= {numel}")


class Payload:
    """Compressed KV rows of one layer, row r = token * H_kv + kv_head
    (ref:src/khq/runtime.mojo:414-425)."""

    def __init__(self, rows: int, device="cuda"):
        self.rows = rows
        z = dict(device=device)
        self.kmask = torch.zeros((rows, 16), dtype=torch.int32, **z)  # u32 bits
        self.kpay = torch.zeros((rows, 40), dtype=torch.uint8, **z)
        self.knorm = torch.zeros(rows, dtype=torch.float16, **z)
        self.krn = torch.zeros(rows, dtype=torch.float16, **z)
        self.vpay = torch.zeros((rows, 104), dtype=torch.uint8, **z)
        self.vnorm = torch.zeros(rows, dtype=torch.float16, **z)
        self.vrn = torch.zeros(rows, dtype=torch.float16, **z)
        self.vsm = torch.zeros((rows, 4), dtype=torch.uint8, **z)

    def tensors(self):
        return (self.kmask, self.kpay, self.knorm, self.krn, self.vpay, self.vnorm, self.vrn,
                self.vsm)

    def nbytes_per_row(self) -> int:
        return ROW_BYTES


class Centroids:
    """Per-layer constant tensors on device (fp16), from a LayerCentroids."""

    def __init__(self, lc, device="cuda"):
        h = lc.fp16()
        self.layer_id = lc.layer_id
        self.ts_k, self.alpha_k = float(lc.ts_k), float(lc.alpha_k)
        self.ts_v, self.alpha_v = float(lc.ts_v), float(lc.alpha_v)
        for k, v in h.items():
            setattr(self, k, torch.from_numpy(v).to(device))


def compress(x: torch.Tensor, cents: Centroids, pay: Payload, row0: int, *, is_v: bool,
             stream=None) -> None:
    """launch_khq_compress_fp16 on rows [row0, row0 + n) of `pay` (x f16 [n, 256])."""
    _need(x, torch.float16, name="x")
    if x.dim() != 2 or x.shape[1] != D:
        raise ValueError(f"x must be [n, {D}]")
    n = x.shape[0]
    if row0 < 0 or row0 + n > pay.rows:
        raise ValueError("compress rows out of payload range")
    if is_v:
        args = (ptr(x), ptr(cents.d_v), ptr(cents.rotor_v), ptr(cents.cents_v), ptr(cents.vq),
                ptr(pay.kmask[row0]), ptr(pay.vnorm[row0:]), ptr(pay.vrn[row0:]),
                ptr(pay.vpay[row0]), ptr(pay.vsm[row0]), n, D, cents.ts_v, cents.alpha_v, 1)
    else:
        args = (ptr(x), ptr(cents.d_k), ptr(cents.rotor_k), ptr(cents.cents_k),
                ptr(cents.cents_k), ptr(pay.kmask[row0]), ptr(pay.knorm[row0:]),
                ptr(pay.krn[row0:]), ptr(pay.kpay[row0]), ptr(pay.vsm[row0]), n, D, cents.ts_k,
                cents.alpha_k, 0)
    call("launch_khq_compress_fp16", *args, stream_handle(stream))


def attn(q_gate: torch.Tensor, pay: Payload, cents: Centroids, out_attn: torch.Tensor, *,
         c_len: int, H_q: int, H_kv: int, scale: float, num_splits: int = 1,
         out_partial: torch.Tensor | None = None, rope_base: float = 1e7, start_pos: int = 0,
         L_q: int = 1, check: bool = True, stream=None) -> int:
    """launch_khq_attn_fp16 (ref call site: src/khq/runtime.mojo:563-586)."""
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    _need(out_attn, torch.float32, H_q * L_q * (D + 2), "out_attn")
    if c_len > 0 and c_len * H_kv > pay.rows:
        raise ValueError("c_len exceeds payload rows")
    n_rep = H_q // H_kv if H_kv > 0 else 0
    return call("launch_khq_attn_fp16", ptr(q_gate), ptr(pay.kpay), ptr(pay.vpay),
                ptr(pay.vsm), ptr(pay.kmask), ptr(pay.knorm), ptr(pay.krn), ptr(pay.vnorm),
                ptr(pay.vrn), ptr(cents.cents_k), ptr(cents.cents_v), ptr(cents.vq),
                ptr(cents.rotor_k), ptr(cents.rotor_v), ptr(cents.d_k), ptr(cents.d_v),
                ptr(out_attn), ptr(out_partial), H_q * L_q, H_q, L_q, c_len, c_len, n_rep,
                scale, cents.alpha_k, cents.alpha_v, rope_base, start_pos, num_splits,
                stream_handle(stream), check=check)


def window_attn(q_gate, ring_k, ring_v, out_attn, *, win_start: int, win_len: int,
                ring_cap: int, H_q: int, H_kv: int, scale: float, check: bool = True,
                stream=None) -> int:
    """launch_khq_window_attn_fp16 (ref call site: src/khq/runtime.mojo:592-603)."""
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    _need(ring_k, torch.float16, ring_cap * H_kv * D, "ring_k")
    _need(ring_v, torch.float16, ring_cap * H_kv * D, "ring_v")
    _need(out_attn, torch.float32, H_q * (D + 2), "out_attn")
    return call("launch_khq_window_attn_fp16", ptr(q_gate), ptr(ring_k), ptr(ring_v),
                ptr(out_attn), win_start, win_len, ring_cap, H_q, H_kv, D, scale,
                stream_handle(stream), check=check)


def merge_gate(attn_c, attn_w, q_gate, out, *, H_q: int, has_w: bool, has_c: bool = True,
               stream=None) -> int:
    """launch_khq_merge_gate_fp16 with the has_c/has_w mapping of
    ref:src/ops.mojo:1255-1279 (has_c false: attn_w stands in for attn_c)."""
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    _need(out, torch.float16, H_q * D, "out")
    src_c = attn_c if has_c else attn_w
    return call("launch_khq_merge_gate_fp16", ptr(src_c), ptr(attn_w), ptr(q_gate), ptr(out),
                H_q, D, 1 if (has_w and has_c) else 0, stream_handle(stream))


def gather_q(q_gate, q_out, *, H_q: int, stream=None) -> int:
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    _need(q_out, torch.float16, H_q * D, "q_out")
    return call("launch_khq_gather_q_fp16", ptr(q_gate), ptr(q_out), H_q, D,
                stream_handle(stream))


def ring_write(ring_k, ring_v, ring_u, k_roped, v, k_unroped, *, slot: int, kv: int,
               stream=None) -> int:
    for name, r, s in (("ring_k", ring_k, k_roped), ("ring_v", ring_v, v),
                       ("ring_u", ring_u, k_unroped)):
        if r is not None:
            _need(r, torch.float16, (slot + 1) * kv, name)
            _need(s, torch.float16, kv, name + " source")
    return call("launch_khq_ring_write_fp16", ptr(ring_k), ptr(ring_v), ptr(ring_u),
                ptr(k_roped), ptr(v), ptr(k_unroped), slot, kv, stream_handle(stream))


def partial_rope(vec, *, num_heads: int, head_dim: int = D, rotary_dim: int = 64, pos: int,
                 theta: float = 1e7, stride: int = 0, stream=None) -> int:
    es = stride if stride > 0 else head_dim
    _need(vec, torch.float16, (num_heads - 1) * es + head_dim, "vec")
    return call("launch_khq_partial_rope_fp16", ptr(vec), num_heads, head_dim, rotary_dim, pos,
                theta, stride, stream_handle(stream))


def gqa_attn(q_gate, k_cache, v_cache, out, *, seq_len: int, H_q: int, H_kv: int,
             head_dim: int = D, scale: float, check: bool = True, stream=None) -> int:
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    _need(k_cache, torch.float16, seq_len * H_kv * D, "k_cache")
    _need(v_cache, torch.float16, seq_len * H_kv * D, "v_cache")
    _need(out, torch.float16, H_q * D, "out")
    return call("launch_khq_gqa_attn_fp16", ptr(q_gate), ptr(k_cache), ptr(v_cache), ptr(out),
                seq_len, H_q, H_kv, head_dim, scale, stream_handle(stream), check=check)


def attn_step(q_gate, pay: Payload, cents: Centroids, ring_k, ring_v, out, *, H_q: int,
              H_kv: int, c_len: int, win_start: int, win_len: int, ring_cap: int,
              scale: float, rope_base: float = 1e7, check: bool = True, stream=None,
              noalloc: bool = False) -> int:
    """khq_attn_step_fp16: both regions + merge + gate in one library call
    (noalloc: khq_attn_step_noalloc_fp16, partials in the library's fixed
    device array instead of its growable workspace)."""
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    _need(out, torch.float16, H_q * D, "out")
    if c_len * H_kv > pay.rows:
        raise ValueError("c_len exceeds payload rows")
    if win_len > 0:
        _need(ring_k, torch.float16, ring_cap * H_kv * D, "ring_k")
        _need(ring_v, torch.float16, ring_cap * H_kv * D, "ring_v")
    name = "khq_attn_step_noalloc_fp16" if noalloc else "khq_attn_step_fp16"
    return call(name, ptr(q_gate), ptr(pay.kpay), ptr(pay.vpay), ptr(pay.vsm),
                ptr(pay.kmask), ptr(pay.knorm), ptr(pay.krn), ptr(pay.vnorm), ptr(pay.vrn),
                ptr(cents.cents_k), ptr(cents.cents_v), ptr(cents.vq), ptr(cents.rotor_k),
                ptr(cents.rotor_v), ptr(cents.d_k), ptr(cents.d_v), ptr(ring_k), ptr(ring_v),
                ptr(out), H_q, H_kv, c_len, win_start, win_len, ring_cap, scale,
                cents.alpha_k, cents.alpha_v, rope_base, stream_handle(stream), check=check)


def attn_step_batched(seqs, cents: Centroids, *, H_q: int, H_kv: int, scale: float,
                      rope_base: float = 1e7, check: bool = True, stream=None) -> int:
    """khq_attn_step_batched_fp16 over a list of per-sequence dicts with keys
    q_gate, pay (Payload), ring_k, ring_v, out, c_len, win_start, win_len,
    ring_cap: every sequence's attention step in one library call."""
    arr = (_lib.KhqSeq * len(seqs))()
    for i, s in enumerate(seqs):
        pay = s["pay"]
        _need(s["q_gate"], torch.float16, H_q * 2 * D, "q_gate")
        _need(s["out"], torch.float16, H_q * D, "out")
        if s["c_len"] * H_kv > pay.rows:
            raise ValueError("c_len exceeds payload rows")
        if s["win_len"] > 0:
            _need(s["ring_k"], torch.float16, s["ring_cap"] * H_kv * D, "ring_k")
            _need(s["ring_v"], torch.float16, s["ring_cap"] * H_kv * D, "ring_v")
        arr[i] = _lib.KhqSeq(ptr(s["q_gate"]), ptr(pay.kpay), ptr(pay.vpay), ptr(pay.vsm),
                             ptr(pay.kmask), ptr(pay.knorm), ptr(pay.krn), ptr(pay.vnorm),
                             ptr(pay.vrn), ptr(s["ring_k"]), ptr(s["ring_v"]), ptr(s["out"]),
                             s["c_len"], s["win_start"], s["win_len"], s["ring_cap"])
    return call("khq_attn_step_batched_fp16", ctypes.cast(arr, ctypes.c_void_p), len(seqs), ptr(cents.cents_k),
                ptr(cents.cents_v), ptr(cents.vq), ptr(cents.rotor_k), ptr(cents.rotor_v),
                ptr(cents.d_k), ptr(cents.d_v), H_q, H_kv, scale, cents.alpha_k, cents.alpha_v,
                rope_base, stream_handle(stream), check=check)


def vt_ld(n_keys: int) -> int:
    """Leading dimension of a V^T buffer for keys [0, n_keys) (padded to 64)."""
    return (n_keys + 63) // 64 * 64


def decompress(pay: Payload, cents: Centroids, out_k, out_vt, *, H_kv: int, tok0: int,
               n_tok: int, key0: int, ld_vt: int, start_pos: int = 0, rope_base: float = 1e7,
               check: bool = True, stream=None) -> int:
    """khq_decompress_fp16: tokens [tok0, tok0 + n_tok) -> roped K rows
    out_k f16 [keys][H_kv][256] at key0.. and V^T out_vt f16 [H_kv][256][ld_vt]."""
    if (tok0 + n_tok) * H_kv > pay.rows:
        raise ValueError("tokens exceed payload rows")
    _need(out_k, torch.float16, (key0 + n_tok) * H_kv * D, "out_k")
    _need(out_vt, torch.float16, H_kv * D * ld_vt, "out_vt")
    return call("khq_decompress_fp16", ptr(pay.kpay), ptr(pay.vpay), ptr(pay.vsm), ptr(pay.kmask),
                ptr(pay.knorm), ptr(pay.krn), ptr(pay.vnorm), ptr(pay.vrn), ptr(cents.cents_k),
                ptr(cents.cents_v), ptr(cents.vq), ptr(cents.rotor_k), ptr(cents.rotor_v),
                ptr(cents.d_k), ptr(cents.d_v), H_kv, tok0, n_tok, start_pos, cents.alpha_k,
                cents.alpha_v, rope_base, ptr(out_k), key0, ptr(out_vt), ld_vt,
                stream_handle(stream), check=check)


def prefill_attn(q_gate, k, vt, out, *, ld_vt: int, n_k: int, n_q: int, vis0: int, H_q: int,
                 H_kv: int, scale: float, check: bool = True, stream=None) -> int:
    """khq_prefill_attn_fp16: n_q queries (q_gate f16 [n_q][H_q][512]) over
    dense keys; query j sees keys [0, vis0 + j); out f16 [n_q][H_q][256] gated."""
    _need(q_gate, torch.float16, n_q * H_q * 2 * D, "q_gate")
    _need(k, torch.float16, n_k * H_kv * D, "k")
    _need(vt, torch.float16, H_kv * D * ld_vt, "vt")
    _need(out, torch.float16, n_q * H_q * D, "out")
    return call("khq_prefill_attn_fp16", ptr(q_gate), ptr(k), ptr(vt), ld_vt, n_k, n_q, vis0,
                H_q, H_kv, scale, ptr(out), stream_handle(stream), check=check)


def prefill_attn_partials(q_gate, k, vt, *, ld_vt: int, n_k: int, n_q: int, vis0: int, H_q: int,
                          H_kv: int, scale: float, check: bool = True, stream=None) -> int:
    """khq_prefill_attn_partials_fp16: the prefill attention kernel alone
    (split partials into the library workspace; profiling)."""
    _need(q_gate, torch.float16, n_q * H_q * 2 * D, "q_gate")
    _need(k, torch.float16, n_k * H_kv * D, "k")
    _need(vt, torch.float16, H_kv * D * ld_vt, "vt")
    return call("khq_prefill_attn_partials_fp16", ptr(q_gate), ptr(k), ptr(vt), ld_vt, n_k, n_q,
                vis0, H_q, H_kv, scale, stream_handle(stream), check=check)


def attn_partials(q_gate, pay: Payload, cents: Centroids, *, H_q: int, H_kv: int, c_len: int,
                  scale: float, rope_base: float = 1e7, stream=None) -> int:
    """khq_attn_partials_fp16: the compressed-region kernel alone (profiling)."""
    _need(q_gate, torch.float16, H_q * 2 * D, "q_gate")
    if c_len * H_kv > pay.rows:
        raise ValueError("c_len exceeds payload rows")
    return call("khq_attn_partials_fp16", ptr(q_gate), ptr(pay.kpay), ptr(pay.vpay),
                ptr(pay.vsm), ptr(pay.kmask), ptr(pay.knorm), ptr(pay.krn), ptr(pay.vnorm),
                ptr(pay.vrn), ptr(cents.cents_k), ptr(cents.cents_v), ptr(cents.vq),
                ptr(cents.rotor_k), ptr(cents.rotor_v), ptr(cents.d_k), ptr(cents.d_v), H_q,
                H_kv, c_len, scale, cents.alpha_k, cents.alpha_v, rope_base,
                stream_handle(stream))


def attn_parts(c_len: int) -> int:
    return int(_lib.lib().khq_attn_parts(c_len))


def workspace_reserve(nbytes: int) -> None:
    call("khq_workspace_reserve", nbytes)


def attn_reduce(partial, out_attn, *, num_queries: int, num_splits: int, stream=None,
                check: bool = True) -> int:
    """khq_attn_reduce_f32: logsumexp merge of split triples (the reduce
    launch_khq_attn_fp16 issues for num_splits > 1)."""
    _need(partial, torch.float32, num_queries * num_splits * (D + 2), "partial")
    _need(out_attn, torch.float32, num_queries * (D + 2), "out_attn")
    return call("khq_attn_reduce_f32", ptr(partial), ptr(out_attn), num_queries, num_splits,
                stream_handle(stream), check=check)


def fault_status(clear: bool = True) -> int:
    """khq_fault_status: nonzero when a hand-off wait of the compressed-region
    kernel gave up since the last clear (those blocks wrote NaN maxima)."""
    v = ctypes.c_int(0)
    call("khq_fault_status", ctypes.addressof(v), 1 if clear else 0)
    return v.value


def set_spin_limit(sleeps: int) -> None:
    """Test knob: bound of the kernel's hand-off waits (0 = default 2^20)."""
    call("khq_set_spin_limit", sleeps)
