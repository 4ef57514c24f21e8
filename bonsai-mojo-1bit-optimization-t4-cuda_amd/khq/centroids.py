"""KHQK v2 centroid file: reader, writer, validator and synthetic generator.

File layout (f32 little-endian), as written by ref:src/khq/calib.mojo:323-329,
524-542 and read by ref:src/khq/runtime.mojo:312-392:

    header  u32 magic 0x4B51484B ('KHQK'), u32 version 2, u32 n_layers, u32 D=256
    per layer:
        u32 layer_id
        f32 ts_k, alpha_k
        f32 d_k[256]              (+-1, make_d)
        f32 cents_k[4][256]       K-static pattern [0, -c, +c, +c]
        f32 rotor_k[64][16]       rotor[p*16 + k*4 + c]
        f32 ts_v, alpha_v
        f32 d_v[256]              (+-1, make_d_v)
        f32 cents_v[4][256]
        f32 rotor_v[64][16]
        f32 vq[64][256][3]

On load the tensors become fp16, as the reference uploads them
(ref:src/khq/runtime.mojo:299-309).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = 0x4B51484B
VERSION = 2
D = 256
NP = 64
MAX_LAYERS = 64  # ref:src/khq/runtime.mojo:35 KHQ_MAX_LAYERS
LAYER_F32 = 2 + D + 4 * D + NP * 16 + 2 + D + 4 * D + NP * 16 + NP * 256 * 3
LAYER_BYTES = 4 + 4 * LAYER_F32


class CentroidFileError(ValueError):
    pass


@dataclass
class LayerCentroids:
    layer_id: int
    ts_k: float = 1.0
    alpha_k: float = 1.0
    d_k: np.ndarray = field(default_factory=lambda: np.ones(D, np.float32))
    cents_k: np.ndarray = field(default_factory=lambda: np.zeros((4, D), np.float32))
    rotor_k: np.ndarray = field(default_factory=lambda: identity_rotors())
    ts_v: float = 1.95  # ref:src/khq/runtime.mojo:124 default
    alpha_v: float = 1.0
    d_v: np.ndarray = field(default_factory=lambda: np.ones(D, np.float32))
    cents_v: np.ndarray = field(default_factory=lambda: np.zeros((4, D), np.float32))
    rotor_v: np.ndarray = field(default_factory=lambda: identity_rotors())
    vq: np.ndarray = field(default_factory=lambda: np.zeros((NP, 256, 3), np.float32))

    def fp16(self) -> dict:
        """The per-layer tensors as the kernels consume them (fp16, flat)."""
        h = lambda a: np.ascontiguousarray(np.asarray(a, np.float32).reshape(-1).astype(np.float16))
        return {
            "d_k": h(self.d_k), "cents_k": h(self.cents_k), "rotor_k": h(self.rotor_k),
            "d_v": h(self.d_v), "cents_v": h(self.cents_v), "rotor_v": h(self.rotor_v),
            "vq": h(self.vq),
        }


def identity_rotors() -> np.ndarray:
    r = np.zeros((NP, 16), np.float32)
    for k in range(4):
        r[:, k * 4 + k] = 1.0
    return r


def _xorshift_d(seed: int) -> np.ndarray:
    s = seed & 0xFFFFFFFF
    out = np.empty(D, np.float32)
    for i in range(D):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = 1.0 if (s & 1) == 1 else -1.0
    return out


def make_d(layer_id: int) -> np.ndarray:
    """K sign vector, ref:src/khq/calib.mojo:137-143 (u32 arithmetic)."""
    return _xorshift_d((layer_id * 2654435761 + 12345) & 0xFFFFFFFF)


def make_d_v(layer_id: int) -> np.ndarray:
    """V sign vector, ref:src/khq/calib.mojo:197-203."""
    return _xorshift_d((layer_id * 40503 + 987654321) & 0xFFFFFFFF)


def quaternion_rotors(rng: np.random.Generator) -> np.ndarray:
    """64 random unit quaternions as 4x4 left-multiplication matrices,
    stored rotor[p*16 + k*4 + c] = L(q)[k][c] (orthogonal)."""
    q = rng.standard_normal((NP, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    a, b, c, d = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    L = np.stack([
        np.stack([a, -b, -c, -d], 1),
        np.stack([b, a, -d, c], 1),
        np.stack([c, d, a, -b], 1),
        np.stack([d, -c, b, a], 1),
    ], 1)  # [NP, 4(k), 4(c)]
    return L.reshape(NP, 16).astype(np.float32)


def synthetic_layer(layer_id: int, seed: int = 1234, ts_k: float = 1.0, alpha_k: float = 1.0,
                    ts_v: float = 1.95, alpha_v: float = 1.0) -> LayerCentroids:
    """Seeded synthetic centroids for one layer.

    d_k/d_v from the reference generators; K cents in the K-static pattern
    [0, -c, +c, +c] with c = 0.935 * sigma * ts_k (sigma = f_s = 1/16, the
    per-dim std of a unit row after FWHT/16); V cents rows [-c_v, +c_v, 0, 0]
    with c_v = 0.8 * sigma, a binary quantizer for patch dim 3; rotors are
    seeded random unit quaternions; the VQ codebook is N(0,1)."""
    rng = np.random.default_rng([seed, layer_id])
    sigma = 1.0 / 16.0
    c = 0.935 * sigma * ts_k
    cents_k = np.zeros((4, D), np.float32)
    cents_k[1] = -c
    cents_k[2] = c
    cents_k[3] = c
    cv = 0.8 * sigma
    cents_v = np.zeros((4, D), np.float32)
    cents_v[0] = -cv
    cents_v[1] = cv
    return LayerCentroids(
        layer_id=layer_id, ts_k=ts_k, alpha_k=alpha_k, d_k=make_d(layer_id), cents_k=cents_k,
        rotor_k=quaternion_rotors(rng), ts_v=ts_v, alpha_v=alpha_v, d_v=make_d_v(layer_id),
        cents_v=cents_v, rotor_v=quaternion_rotors(rng),
        vq=rng.standard_normal((NP, 256, 3)).astype(np.float32))


def write(path: str, layers: list[LayerCentroids]) -> None:
    with open(path, "wb") as f:
        f.write(struct.pack("<IIII", MAGIC, VERSION, len(layers), D))
        for L in layers:
            f.write(struct.pack("<I", L.layer_id))
            f.write(struct.pack("<ff", L.ts_k, L.alpha_k))
            for a in (L.d_k, L.cents_k, L.rotor_k):
                f.write(np.asarray(a, "<f4").reshape(-1).tobytes())
            f.write(struct.pack("<ff", L.ts_v, L.alpha_v))
            for a in (L.d_v, L.cents_v, L.rotor_v, L.vq):
                f.write(np.asarray(a, "<f4").reshape(-1).tobytes())


def read(path: str) -> dict[int, LayerCentroids]:
    """Parses a KHQK v2 file like ref:src/khq/runtime.mojo:312-392: rejects a
    short file or bad magic, version != 2 and layer_id outside [0, 64); also
    rejects a truncated layer block, which the reference would read past."""
    with open(path, "rb") as f:
        buf = f.read()
    if len(buf) < 16:
        raise CentroidFileError(f"{path}: file too short ({len(buf)} bytes)")
    magic, ver, n_layers, dim = struct.unpack_from("<IIII", buf, 0)
    if magic != MAGIC:
        raise CentroidFileError(f"{path}: bad magic {magic:#x}")
    if ver != VERSION:
        raise CentroidFileError(f"{path}: unsupported version {ver}")
    if dim != D:
        raise CentroidFileError(f"{path}: D={dim}, only 256 is supported")
    off = 16
    out: dict[int, LayerCentroids] = {}
    for li in range(n_layers):
        if off + LAYER_BYTES > len(buf):
            raise CentroidFileError(f"{path}: truncated at layer index {li}")
        (layer_id,) = struct.unpack_from("<I", buf, off)
        off += 4
        if not 0 <= layer_id < MAX_LAYERS:
            raise CentroidFileError(f"{path}: layer_id {layer_id} out of range")

        def take(n):
            nonlocal off
            a = np.frombuffer(buf, "<f4", n, off).astype(np.float32)
            off += 4 * n
            return a

        ts_k, alpha_k = take(2)
        d_k, cents_k, rotor_k = take(D), take(4 * D).reshape(4, D), take(NP * 16).reshape(NP, 16)
        ts_v, alpha_v = take(2)
        d_v, cents_v = take(D), take(4 * D).reshape(4, D)
        rotor_v = take(NP * 16).reshape(NP, 16)
        vq = take(NP * 256 * 3).reshape(NP, 256, 3)
        out[layer_id] = LayerCentroids(layer_id, float(ts_k), float(alpha_k), d_k, cents_k,
                                       rotor_k, float(ts_v), float(alpha_v), d_v, cents_v,
                                       rotor_v, vq)
    return out


def validate(path: str) -> list[str]:
    """The deploy gate's checks on a centroid file
    (ref:deploy_on_kaggle.sh:1507-1537): magic, finite and |v| <= 1e6,
    0.05 < ts < 1000, |d_k[:16]| == 1, exact size.  Returns the problems."""
    problems: list[str] = []
    with open(path, "rb") as f:
        buf = f.read()
    if len(buf) < 16:
        return ["file too short"]
    magic, ver, nl, dim = struct.unpack_from("<IIII", buf, 0)
    if magic != MAGIC:
        return [f"bad magic {magic:#x}"]
    off = 16
    for _ in range(nl):
        if off + LAYER_BYTES > len(buf):
            problems.append("truncated")
            return problems
        (lid,) = struct.unpack_from("<I", buf, off)
        off += 4
        ts_k, _ak = struct.unpack_from("<ff", buf, off)
        off += 8
        vals = []
        for n in (D, 4 * D, NP * 16):
            vals.append(np.frombuffer(buf, "<f4", n, off))
            off += 4 * n
        ts_v, _av = struct.unpack_from("<ff", buf, off)
        off += 8
        for n in (D, 4 * D, NP * 16, NP * 768):
            vals.append(np.frombuffer(buf, "<f4", n, off))
            off += 4 * n
        for v in vals:
            if not np.all(np.isfinite(v)) or np.any(np.abs(v) > 1e6):
                problems.append(f"layer {lid}: non-finite or huge values")
                break
        if not (0.05 < ts_k < 1000 and 0.05 < ts_v < 1000):
            problems.append(f"layer {lid}: threshold scale out of range")
        if np.any(np.abs(vals[0][:16]) != 1.0):
            problems.append(f"layer {lid}: d_k not +-1")
    if off != len(buf):
        problems.append(f"{len(buf) - off} trailing bytes")
    return problems
