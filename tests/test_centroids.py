"""KHQK v2 centroid files: write/read round trip, the deploy validator and
the loader's rejections (ref:src/khq/runtime.mojo:312-392,
ref:deploy_on_kaggle.sh:1507-1537)."""
import struct

import numpy as np
import pytest

from khq import centroids as C


def test_make_d_generators():
    # xorshift32 restated with numpy uint32 ops (independent of the Python ints)
    def ref(seed):
        s = np.uint32(seed)
        out = []
        with np.errstate(over="ignore"):
            for _ in range(256):
                s ^= np.uint32(s << np.uint32(13))
                s ^= np.uint32(s >> np.uint32(17))
                s ^= np.uint32(s << np.uint32(5))
                out.append(1.0 if s & 1 else -1.0)
        return np.array(out, np.float32)

    for lid in (0, 3, 15, 63):
        seed_k = (lid * 2654435761 + 12345) & 0xFFFFFFFF
        seed_v = (lid * 40503 + 987654321) & 0xFFFFFFFF
        assert np.array_equal(C.make_d(lid), ref(seed_k))
        assert np.array_equal(C.make_d_v(lid), ref(seed_v))
        assert set(np.unique(C.make_d(lid))) <= {-1.0, 1.0}
    assert not np.array_equal(C.make_d(3), C.make_d(4))


def test_rotors_orthogonal():
    r = C.quaternion_rotors(np.random.default_rng(0)).reshape(64, 4, 4).astype(np.float64)
    for p in range(64):
        np.testing.assert_allclose(r[p] @ r[p].T, np.eye(4), atol=1e-6)


def test_roundtrip_and_validate(tmp_path):
    layers = [C.synthetic_layer(i) for i in (0, 3, 15)]
    path = tmp_path / "khq_calib.bin"
    C.write(str(path), layers)
    assert path.stat().st_size == 16 + 3 * C.LAYER_BYTES
    assert C.validate(str(path)) == []
    got = C.read(str(path))
    assert sorted(got) == [0, 3, 15]
    for L in layers:
        g = got[L.layer_id]
        for name in ("d_k", "cents_k", "rotor_k", "d_v", "cents_v", "rotor_v", "vq"):
            assert np.array_equal(getattr(g, name), np.asarray(getattr(L, name), np.float32))
        assert g.ts_v == pytest.approx(1.95)


def _bytes(tmp_path, layers=1):
    path = tmp_path / "f.bin"
    C.write(str(path), [C.synthetic_layer(i) for i in range(layers)])
    return path, bytearray(path.read_bytes())


def test_rejections(tmp_path):
    path, b = _bytes(tmp_path)
    bad = tmp_path / "bad.bin"
    bad.write_bytes(bytes(b[:10]))
    with pytest.raises(C.CentroidFileError):
        C.read(str(bad))
    b2 = bytearray(b)
    b2[0:4] = struct.pack("<I", 0x12345678)
    bad.write_bytes(bytes(b2))
    with pytest.raises(C.CentroidFileError, match="magic"):
        C.read(str(bad))
    assert C.validate(str(bad)) != []
    b2 = bytearray(b)
    b2[4:8] = struct.pack("<I", 1)
    bad.write_bytes(bytes(b2))
    with pytest.raises(C.CentroidFileError, match="version"):
        C.read(str(bad))
    b2 = bytearray(b)
    b2[16:20] = struct.pack("<I", 64)
    bad.write_bytes(bytes(b2))
    with pytest.raises(C.CentroidFileError, match="out of range"):
        C.read(str(bad))
    bad.write_bytes(bytes(b[:-8]))
    with pytest.raises(C.CentroidFileError, match="truncated"):
        C.read(str(bad))
    assert "truncated" in C.validate(str(bad))


def test_validator_checks_values(tmp_path):
    L = C.synthetic_layer(0)
    L.ts_k = 0.01
    p = tmp_path / "v.bin"
    C.write(str(p), [L])
    assert any("threshold" in m for m in C.validate(str(p)))
    L = C.synthetic_layer(0)
    L.vq[0, 0, 0] = np.nan
    C.write(str(p), [L])
    assert any("non-finite" in m for m in C.validate(str(p)))
