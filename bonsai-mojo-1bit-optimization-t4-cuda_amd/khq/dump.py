"""Calibration dumps: the KHQD (K/V activations) and KHQA (attention scores)
files of ref:src/models/qwen3_5/khq_dump.mojo.

`Recorder` drives the native recorder (khq_dump_* in include/khq.h): K/V
rows accumulate on the GPU and are written by `flush`; attention scores are
computed on the GPU per token and appended to attn_<layer>.bin.  The readers
are plain numpy over the byte layouts, for the calibration and for tests:

  kv_dump.bin   u32 'KHQD' | u32 n_layers | u32 dim | n_layers x (u32 layer_id,
                u32 n_tokens) | per layer K f32 [n][dim] then V f32 [n][dim]
                (khq_dump.mojo:9-14, 319-368)
  attn_<l>.bin  u32 'KHQA' | u32 H_q | u32 H_kv | u32 D | per token u32 n_valid
                then fp16 [H_q][n_valid] (khq_dump.mojo:87-93, 199-316)
"""
from __future__ import annotations

import os
import struct

import numpy as np

MAGIC_KV = 0x4451484B    # 'KHQD'
MAGIC_ATTN = 0x4151484B  # 'KHQA'
DUMP_KV, DUMP_ATTN = 1, 2


def read_kv_dump(path: str) -> dict[int, tuple[np.ndarray, np.ndarray]]:
    """kv_dump.bin -> {layer_id: (K f32 [n, dim], V f32 [n, dim])}, in file
    order; raises ValueError on a bad magic or a truncated file (the checks
    of ref:src/khq/calib.mojo:400-440)."""
    buf = np.fromfile(path, dtype=np.uint8)
    if buf.size < 12:
        raise ValueError(f"{path}: {buf.size} bytes, no KHQD header")
    magic, n_layers, dim = struct.unpack_from("<III", buf, 0)
    if magic != MAGIC_KV:
        raise ValueError(f"{path}: magic {magic:#x} is not KHQD")
    if n_layers < 1 or dim < 1 or 12 + 8 * n_layers > buf.size:
        raise ValueError(f"{path}: header table truncated ({n_layers} layers)")
    table = [struct.unpack_from("<II", buf, 12 + 8 * i) for i in range(n_layers)]
    off = 12 + 8 * n_layers
    out = {}
    for layer_id, n in table:
        nb = n * dim * 4
        if off + 2 * nb > buf.size:
            raise ValueError(f"{path}: layer {layer_id} truncated")
        k = buf[off:off + nb].view("<f4").reshape(n, dim)
        v = buf[off + nb:off + 2 * nb].view("<f4").reshape(n, dim)
        out[layer_id] = (k, v)
        off += 2 * nb
    return out


def write_kv_dump(path: str, layers: dict[int, tuple[np.ndarray, np.ndarray]]) -> None:
    """The KHQD layout from host arrays (tests, synthetic calibration inputs)."""
    ids = sorted(layers)
    dim = layers[ids[0]][0].shape[1]
    with open(path, "wb") as f:
        f.write(struct.pack("<III", MAGIC_KV, len(ids), dim))
        for i in ids:
            f.write(struct.pack("<II", i, layers[i][0].shape[0]))
        for i in ids:
            k, v = layers[i]
            f.write(np.ascontiguousarray(k, "<f4").tobytes())
            f.write(np.ascontiguousarray(v, "<f4").tobytes())


def read_attn_dump(path: str):
    """attn_<layer>.bin -> (H_q, H_kv, D, records), records = list of fp16
    arrays [H_q, n_valid] in token order."""
    buf = np.fromfile(path, dtype=np.uint8)
    if buf.size < 16:
        raise ValueError(f"{path}: no KHQA header")
    magic, H_q, H_kv, D = struct.unpack_from("<IIII", buf, 0)
    if magic != MAGIC_ATTN:
        raise ValueError(f"{path}: magic {magic:#x} is not KHQA")
    recs, off = [], 16
    while off + 4 <= buf.size:
        (nv,) = struct.unpack_from("<I", buf, off)
        nb = H_q * nv * 2
        if off + 4 + nb > buf.size:
            raise ValueError(f"{path}: record {len(recs)} truncated")
        recs.append(buf[off + 4:off + 4 + nb].view("<f2").reshape(H_q, nv))
        off += 4 + nb
    return H_q, H_kv, D, recs


def attn_matrix(path: str) -> np.ndarray:
    """The calibration's view of attn_<layer>.bin: f32 [H_q, T, T] with row t
    holding token t's scores over keys 0..n_valid-1 and zeros after
    (ref:src/khq/calib.mojo:249-291)."""
    H_q, _, _, recs = read_attn_dump(path)
    T = len(recs)
    out = np.zeros((H_q, T, T), np.float32)
    for t, r in enumerate(recs):
        nv = min(r.shape[1], T)
        out[:, t, :nv] = r[:, :nv].astype(np.float32)
    return out


def half_bits_ref(x: np.ndarray) -> np.ndarray:
    """fp16 bits of float32 values the way the reference writes scores
    (khq_dump.mojo:95-117): round-to-nearest-even for normal results,
    round-half-up of (512 + m / 16384) * 2^e for subnormal ones."""
    x = np.asarray(x, np.float32)
    bits = x.view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    ex = ((bits >> 23) & 0xFF) - 127 + 15
    man = bits & 0x7FFFFF
    half = (ex << 10) | (man >> 13)
    rem = man & 0x1FFF
    rne = half + ((rem > 0x1000) | ((rem == 0x1000) & ((half & 1) == 1)))
    with np.errstate(over="ignore", invalid="ignore"):
        sub = np.floor((512.0 + man.astype(np.float64) / 16384.0) *
                       np.ldexp(1.0, np.clip(ex, -40, 0)) + 0.5).astype(np.int64)
    out = np.where(ex >= 31, 0x7C00, np.where(ex > 0, rne, np.where(ex < -9, 0, sub)))
    return (sign | out).astype(np.uint16)


class Recorder:
    """The native dump recorder (khq_dump_create / kv / attn / flush)."""

    def __init__(self, directory: str, max_tokens: int, kv_dim: int,
                 flags: int = DUMP_KV | DUMP_ATTN):
        from . import _lib

        os.makedirs(directory, exist_ok=True)
        self._lib = _lib
        self.handle = _lib.lib().khq_dump_create(directory.encode(), max_tokens, kv_dim, flags)
        if not self.handle:
            raise ValueError("khq_dump_create rejected its arguments")
        self.directory = directory

    def kv(self, layer: int, k, v, stream=None) -> None:
        self._lib.call("khq_dump_kv", self.handle, layer, self._lib.ptr(k), self._lib.ptr(v),
                       self._lib.stream_handle(stream))

    def attn(self, layer: int, q_gate, k_roped, pos: int, *, H_q: int, H_kv: int, D: int,
             scale: float, stream=None) -> None:
        self._lib.call("khq_dump_attn", self.handle, layer, self._lib.ptr(q_gate),
                       self._lib.ptr(k_roped), pos, H_q, H_kv, D, scale,
                       self._lib.stream_handle(stream))

    def count(self, layer: int) -> int:
        return int(self._lib.lib().khq_dump_count(self.handle, layer))

    def flush(self) -> None:
        self._lib.call("khq_dump_flush", self.handle)

    def close(self) -> None:
        if self.handle:
            self._lib.lib().khq_dump_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
