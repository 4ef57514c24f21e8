"""Per-layer KHQ runtime: ring buffer, compression cadence, split count and
the two-region attention step.

Mirrors ref:src/khq/runtime.mojo (KhqLayer :77-152, KhqGlobals :155-173,
khq_init :312-392, khq_init_layer :395-429, khq_capture_unroped :432-451,
khq_step :454-613) with torch device tensors in place of Mojo DeviceBuffers
and libkhq_hip.so in place of libbonsai_qmv_sm75.so.
"""
from __future__ import annotations

import ctypes
import os
import time
from dataclasses import dataclass, field

import torch

from . import centroids as C
from . import ops
from .ops import D, Centroids, Payload

RING = 256          # ref runtime.mojo:36 KHQ_RING
WATERMARK = 256     # :37
CHUNK = 128         # :38
MAX_SPLITS = 32     # :42 (the reference clamp)
MIN_TOKENS_PER_SPLIT = 8  # :43
ROPE_BASE = 10000000.0    # runtime.mojo:582

PHASES = ("ring-write", "compress-K", "compress-V", "attn-compressed", "attn-window",
          "merge+gate")


def _env_int(name: str, fallback: int) -> int:
    v = os.environ.get(name)
    if not v:
        return fallback
    try:
        return int(v)
    except ValueError:
        return fallback


@dataclass
class KhqOptions:
    """Runtime switches.  `splits` follows BONSAI_KHQ_SPLITS (default 16,
    clamped to [1, max_splits]; ref runtime.mojo:378-382).  max_splits is 32
    as in the reference; a caller may raise it (e.g. 64) to pass larger split
    counts through the reference entry point.  `fused` selects the single-call
    two-region step (khq_attn_step_fp16) instead of the reference's
    attn + window + merge sequence."""
    splits: int = 16
    max_splits: int = MAX_SPLITS
    prof: bool = False
    debug: bool = False
    fused: bool = True

    @classmethod
    def from_env(cls, **over) -> "KhqOptions":
        o = cls(**over)
        o.splits = _env_int("BONSAI_KHQ_SPLITS", o.splits)
        o.splits = max(1, min(o.splits, o.max_splits))
        o.prof = os.environ.get("BONSAI_KHQ_PROF", "")[:1] == "1" or o.prof
        o.debug = os.environ.get("BONSAI_KHQ_DEBUG", "")[:1] == "1" or o.debug
        return o


def split_count(c_len: int, splits: int) -> int:
    """ref runtime.mojo:211-222: 1 if splits <= 1 or c_len <= 0, else
    clamp(c_len // 8, 1, splits)."""
    if splits <= 1 or c_len <= 0:
        return 1
    return max(1, min(c_len // MIN_TOKENS_PER_SPLIT, splits))


def plan_step(boundary: int, write_pos: int, cap: int):
    """Host bookkeeping of one step after the ring write (ref runtime.mojo:
    489-590): write_pos advances; a compression event fires when the raw
    window reaches the watermark and boundary + 128 fits the capacity.
    Returns (boundary, write_pos, event_row0_or_None, c_len, win_len, win_start)."""
    write_pos += 1
    event = None
    if write_pos - boundary >= WATERMARK and boundary + CHUNK <= cap:
        event = boundary
        boundary += CHUNK
    c_len = boundary
    win_len = write_pos - c_len
    return boundary, write_pos, event, c_len, win_len, c_len % RING


@dataclass
class CompressEvent:
    boundary: int      # boundary after the event
    write_pos: int
    raw_window: int
    knorm_bits: list = field(default_factory=list)  # fp16 bits of the new K norms (debug)


class KhqLayer:
    """State of one attention layer (all buffers on the device)."""

    def __init__(self, cents: C.LayerCentroids, *, H_q: int = 24, H_kv: int = 4, cap: int = 4096,
                 device="cuda", options: KhqOptions | None = None):
        if H_kv <= 0 or H_q % H_kv != 0:
            raise ValueError("H_q must be a multiple of H_kv")
        self.H_q, self.H_kv, self.D, self.cap = H_q, H_kv, D, cap
        self.device = torch.device(device)
        self.opt = options or KhqOptions.from_env()
        self.cents = Centroids(cents, device)
        kv = H_kv * D
        z = dict(device=self.device, dtype=torch.float16)
        self.ring_k = torch.zeros((RING, H_kv, D), **z)
        self.ring_v = torch.zeros((RING, H_kv, D), **z)
        self.ring_u = torch.zeros((RING, H_kv, D), **z)
        self.kv = kv
        self.pay = Payload(cap * H_kv, device)
        self.ac = torch.zeros((H_q, D + 2), device=self.device, dtype=torch.float32)
        self.aw = torch.zeros((H_q, D + 2), device=self.device, dtype=torch.float32)
        self.ap = torch.zeros((H_q, max(self.opt.max_splits, 1), D + 2), device=self.device,
                              dtype=torch.float32)
        self.boundary = 0
        self.write_pos = 0
        self.events: list[CompressEvent] = []
        self.prof_ns = [0.0] * len(PHASES)

    # ------------------------------------------------------------ state
    def reset(self) -> None:
        """boundary = write_pos = 0 (the reference has no reset, README:260)."""
        self.boundary = 0
        self.write_pos = 0
        self.events.clear()

    def capture_unroped(self, k: torch.Tensor) -> None:
        """Copies post-norm, pre-RoPE K of the token about to be stepped into
        ring_u[write_pos % 256] (ref runtime.mojo:432-451)."""
        slot = self.write_pos % RING
        ops.ring_write(None, None, self.ring_u, None, None, k.reshape(-1), slot=slot,
                       kv=self.kv)

    # ------------------------------------------------------------ step
    def _sync_time(self, phase: int, t0: float) -> float:
        if self.opt.prof:
            torch.cuda.synchronize(self.device)
            t1 = time.perf_counter_ns()
            self.prof_ns[phase] += t1 - t0
            return t1
        return t0

    def step(self, q_gate: torch.Tensor, k_roped: torch.Tensor, v: torch.Tensor,
             out: torch.Tensor, scale: float, k_unroped: torch.Tensor | None = None) -> bool:
        """One decode step of ref runtime.mojo:454-613.  Returns False when
        neither region exists.  If k_unroped is given it is written to
        ring_u in the same launch as K/V (otherwise capture_unroped() must
        have been called for this token)."""
        if self.opt.prof:
            torch.cuda.synchronize(self.device)
        t0 = time.perf_counter_ns()
        slot = self.write_pos % RING
        ops.ring_write(self.ring_k, self.ring_v, self.ring_u if k_unroped is not None else None,
                       k_roped.reshape(-1), v.reshape(-1),
                       k_unroped.reshape(-1) if k_unroped is not None else None,
                       slot=slot, kv=self.kv)
        t0 = self._sync_time(0, t0)
        old_boundary = self.boundary
        _, self.write_pos, event, _, _, _ = plan_step(self.boundary, self.write_pos, self.cap)
        if event is not None:
            s0 = old_boundary % RING
            r0 = old_boundary * self.H_kv
            xk = self.ring_u[s0:s0 + CHUNK].reshape(CHUNK * self.H_kv, D)
            xv = self.ring_v[s0:s0 + CHUNK].reshape(CHUNK * self.H_kv, D)
            ops.compress(xk, self.cents, self.pay, r0, is_v=False)
            t0 = self._sync_time(1, t0)
            ops.compress(xv, self.cents, self.pay, r0, is_v=True)
            t0 = self._sync_time(2, t0)
            bits = []
            if self.opt.debug:
                nb = self.pay.knorm[r0:r0 + CHUNK * self.H_kv].cpu().view(torch.int16)
                bits = [int(b) & 0xFFFF for b in nb.tolist()]
            self.boundary += CHUNK
            self.events.append(CompressEvent(self.boundary, self.write_pos,
                                             self.write_pos - self.boundary, bits))

        c_len = self.boundary
        win_len = self.write_pos - c_len
        has_c, has_w = c_len > 0, win_len > 0
        if not (has_c or has_w):
            return False
        if win_len > RING:
            # ref runtime.mojo:495 skips compression when boundary+128 > cap and
            # then reads overwritten ring slots (README:259); refuse instead.
            raise RuntimeError(f"raw window {win_len} exceeds the {RING}-slot ring "
                               f"(cap {self.cap} reached)")
        win_start = c_len % RING
        if self.opt.fused:
            ops.attn_step(q_gate, self.pay, self.cents, self.ring_k, self.ring_v, out,
                          H_q=self.H_q, H_kv=self.H_kv, c_len=c_len, win_start=win_start,
                          win_len=win_len, ring_cap=RING, scale=scale, rope_base=ROPE_BASE)
            self._sync_time(3, t0)
            return True
        if has_c:
            n_sp = split_count(c_len, self.opt.splits)
            ops.attn(q_gate, self.pay, self.cents, self.ac, c_len=c_len, H_q=self.H_q,
                     H_kv=self.H_kv, scale=scale, num_splits=n_sp,
                     out_partial=self.ap if n_sp > 1 else None, rope_base=ROPE_BASE)
            t0 = self._sync_time(3, t0)
        if has_w:
            ops.window_attn(q_gate, self.ring_k, self.ring_v, self.aw, win_start=win_start,
                            win_len=win_len, ring_cap=RING, H_q=self.H_q, H_kv=self.H_kv,
                            scale=scale)
            t0 = self._sync_time(4, t0)
        ops.merge_gate(self.ac, self.aw, q_gate, out, H_q=self.H_q, has_w=has_w, has_c=has_c)
        self._sync_time(5, t0)
        return True

    def prof_report(self) -> str:
        """Per-phase totals, like khq_prof_report (ref runtime.mojo:232-256)."""
        tot = sum(self.prof_ns)
        lines = [f"[KHQ-PROF] total {tot / 1e6:.3f} ms | splits {self.opt.splits}"]
        for name, ns in zip(PHASES, self.prof_ns):
            pct = 100.0 * ns / tot if tot > 0 else 0.0
            lines.append(f"[KHQ-PROF]   {name:16s} {ns / 1e6:.3f} ms | {pct:.1f} %")
        return "\n".join(lines)

    # ------------------------------------------------- direct state loading
    def load_state(self, *, boundary: int, write_pos: int, rows: dict | None = None,
                   ring_k=None, ring_v=None, ring_u=None) -> None:
        """Installs a prepared state (compressed rows [0, boundary*H_kv) and
        ring contents), for benchmarks and tests that start mid-sequence."""
        if boundary % CHUNK or boundary > self.cap or write_pos < boundary or \
                write_pos - boundary > RING:
            raise ValueError("inconsistent KHQ state")
        self.boundary, self.write_pos = boundary, write_pos
        if rows is not None:
            n = boundary * self.H_kv
            for name in ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm"):
                getattr(self.pay, name)[:n].copy_(rows[name][:n])
        for dst, src in ((self.ring_k, ring_k), (self.ring_v, ring_v), (self.ring_u, ring_u)):
            if src is not None:
                dst.copy_(src.reshape(dst.shape))


class NativeKhqLayer:
    """The same per-layer runtime driven through the C ABI (khq_layer_*): the
    ring, payload, cadence and attention issue all live in libkhq_hip.so; this
    class only holds the handle and the caller-owned constant tensors."""

    def __init__(self, cents: C.LayerCentroids, *, H_q: int = 24, H_kv: int = 4,
                 cap: int = 4096, device="cuda", options: KhqOptions | None = None):
        from . import _lib

        self.opt = options or KhqOptions.from_env()
        self.cents = Centroids(cents, device)
        self.H_q, self.H_kv, self.cap = H_q, H_kv, cap
        c = self.cents
        self._lib = _lib.lib()
        self.handle = self._lib.khq_layer_create(
            H_q, H_kv, cap, c.cents_k.data_ptr(), c.cents_v.data_ptr(), c.vq.data_ptr(),
            c.rotor_k.data_ptr(), c.rotor_v.data_ptr(), c.d_k.data_ptr(), c.d_v.data_ptr(),
            c.ts_k, c.alpha_k, c.ts_v, c.alpha_v, ROPE_BASE, self.opt.splits,
            1 if self.opt.fused else 0)
        if not self.handle:
            raise RuntimeError("khq_layer_create failed")

    def __del__(self):
        h = getattr(self, "handle", None)
        if h:
            self._lib.khq_layer_destroy(h)
            self.handle = None

    def state(self) -> tuple[int, int, int]:
        b, w, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        self._lib.khq_layer_state(self.handle, ctypes.byref(b), ctypes.byref(w), ctypes.byref(n))
        return b.value, w.value, n.value

    def reset(self) -> None:
        self._lib.khq_layer_reset(self.handle)

    def payload_ptrs(self) -> list[int]:
        arr = (ctypes.c_void_p * 11)()
        self._lib.khq_layer_payload(self.handle, arr)
        return [int(p or 0) for p in arr]

    def dense(self) -> tuple[int, int, int, int]:
        """(K rows pointer, V^T pointer, V^T row stride, rows decoded) of the
        prefill path's dense key space."""
        k, vt = ctypes.c_void_p(), ctypes.c_void_p()
        ld, nd = ctypes.c_int(), ctypes.c_int()
        self._lib.khq_layer_dense(self.handle, ctypes.byref(k), ctypes.byref(vt),
                                  ctypes.byref(ld), ctypes.byref(nd))
        return int(k.value or 0), int(vt.value or 0), ld.value, nd.value

    def capture_unroped(self, k: torch.Tensor) -> None:
        from ._lib import KhqError, stream_handle

        rc = self._lib.khq_layer_capture_unroped(self.handle, k.data_ptr(), stream_handle())
        if rc:
            raise KhqError("khq_layer_capture_unroped", rc)

    def step(self, q_gate, k_roped, v, out, scale: float, k_unroped=None) -> bool:
        from ._lib import KhqError, stream_handle

        rc = self._lib.khq_layer_step(self.handle, q_gate.data_ptr(), k_roped.data_ptr(),
                                      v.data_ptr(),
                                      k_unroped.data_ptr() if k_unroped is not None else None,
                                      out.data_ptr(), scale, stream_handle())
        if rc == -102:
            raise RuntimeError(f"raw window exceeds the {RING}-slot ring (cap {self.cap} reached)")
        if rc < 0 or rc > 1:
            raise KhqError("khq_layer_step", rc)
        return rc == 1

    def attention_step(self, q_gate, k, v, out, scale: float, *, pos: int, q_norm_w=None,
                       k_norm_w=None, eps: float = 1e-6) -> bool:
        """khq_layer_attention_step: head RMSNorm of q and k (in place), unroped
        capture, partial RoPE at `pos` (in place), ring writes, dumps, then the
        KHQ step (ref:src/models/qwen3_5/attention.mojo:319-365)."""
        from ._lib import KhqError, stream_handle

        for t, n in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
            if t is not None and (t.dtype != torch.float32 or t.numel() != 256):
                raise ValueError(f"{n} must be float32 [256]")
        rc = self._lib.khq_layer_attention_step(
            self.handle, q_gate.data_ptr(), k.data_ptr(), v.data_ptr(),
            q_norm_w.data_ptr() if q_norm_w is not None else None,
            k_norm_w.data_ptr() if k_norm_w is not None else None, eps, pos, out.data_ptr(),
            scale, stream_handle())
        if rc == -102:
            raise RuntimeError(f"raw window exceeds the {RING}-slot ring (cap {self.cap} reached)")
        if rc < 0 or rc > 1:
            raise KhqError("khq_layer_attention_step", rc)
        return rc == 1

    def set_dump(self, recorder, layer_id: int) -> None:
        """Attach a khq.dump.Recorder (None detaches) for attention_step."""
        from ._lib import KhqError

        rc = self._lib.khq_layer_set_dump(self.handle, recorder.handle if recorder else None,
                                          layer_id)
        if rc:
            raise KhqError("khq_layer_set_dump", rc)
        self._dump = recorder  # keep it alive while attached

    def prefill(self, q_gate, k_roped, v, k_unroped, out, scale: float) -> int:
        """khq_layer_prefill: n tokens at once (q_gate f16 [n][H_q][512], k_roped /
        v / k_unroped f16 [n][H_kv][256], out f16 [n][H_q][256]), the results of
        n steps."""
        from ._lib import KhqError, stream_handle

        n = q_gate.shape[0]
        ops._need(q_gate, torch.float16, n * self.H_q * 2 * D, "q_gate")
        for name, t in (("k_roped", k_roped), ("v", v), ("k_unroped", k_unroped)):
            ops._need(t, torch.float16, n * self.H_kv * D, name)
        ops._need(out, torch.float16, n * self.H_q * D, "out")
        rc = self._lib.khq_layer_prefill(self.handle, ops.ptr(q_gate), ops.ptr(k_roped),
                                         ops.ptr(v), ops.ptr(k_unroped), ops.ptr(out), n, scale,
                                         stream_handle())
        if rc == -102:
            raise RuntimeError("KHQ prefill: raw window would exceed the 256-slot ring")
        if rc != n:
            raise KhqError("khq_layer_prefill", rc)
        return rc


class KhqRuntime:
    """khq_activate / khq_init: loads a KHQK v2 file and creates the layers
    lazily (khq_init_layer is idempotent, ref runtime.mojo:395-429)."""

    def __init__(self, path: str, max_seq: int = 4096, device="cuda",
                 options: KhqOptions | None = None):
        self.centroids = C.read(path)
        self.max_seq = max_seq
        self.device = device
        self.opt = options or KhqOptions.from_env()
        self.layers: dict[int, KhqLayer] = {}

    def layer(self, layer_idx: int, H_q: int = 24, H_kv: int = 4) -> KhqLayer:
        if layer_idx not in self.layers:
            if layer_idx not in self.centroids:
                raise KeyError(f"no centroids for layer {layer_idx}")
            self.layers[layer_idx] = KhqLayer(self.centroids[layer_idx], H_q=H_q, H_kv=H_kv,
                                              cap=self.max_seq, device=self.device,
                                              options=self.opt)
        return self.layers[layer_idx]
