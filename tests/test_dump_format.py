"""KHQD / KHQA byte layouts (ref:src/models/qwen3_5/khq_dump.mojo:9-14, 87-93,
319-368) and the reference's fp16 rounding of scores (:95-117), on the CPU."""
import struct

import numpy as np
import pytest

from khq import dump


def test_kv_dump_roundtrip_and_layout(tmp_path):
    rng = np.random.default_rng(0)
    layers = {3: (rng.standard_normal((5, 1024)).astype(np.float32),
                  rng.standard_normal((5, 1024)).astype(np.float32)),
              7: (rng.standard_normal((2, 1024)).astype(np.float32),
                  rng.standard_normal((2, 1024)).astype(np.float32))}
    p = str(tmp_path / "kv_dump.bin")
    dump.write_kv_dump(p, layers)
    raw = open(p, "rb").read()
    # header: magic, n_layers, dim, then (layer_id, n) pairs, then K, V blocks
    assert struct.unpack_from("<III", raw, 0) == (0x4451484B, 2, 1024)
    assert struct.unpack_from("<IIII", raw, 12) == (3, 5, 7, 2)
    assert len(raw) == 12 + 16 + 2 * (5 + 2) * 1024 * 4
    first_k = np.frombuffer(raw, "<f4", 1024, 28)
    np.testing.assert_array_equal(first_k, layers[3][0][0])
    got = dump.read_kv_dump(p)
    assert list(got) == [3, 7]
    for i in layers:
        np.testing.assert_array_equal(got[i][0], layers[i][0])
        np.testing.assert_array_equal(got[i][1], layers[i][1])


def test_kv_dump_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(struct.pack("<III", 0x12345678, 1, 256))
    with pytest.raises(ValueError, match="magic"):
        dump.read_kv_dump(str(p))
    p.write_bytes(struct.pack("<IIIII", 0x4451484B, 1, 256, 0, 4) + b"\0" * 100)
    with pytest.raises(ValueError, match="truncated"):
        dump.read_kv_dump(str(p))


def test_attn_dump_reader_and_matrix(tmp_path):
    H_q = 3
    p = tmp_path / "attn_2.bin"
    recs = [np.full((H_q, t + 1), 1.0 / (t + 1), np.float16) for t in range(4)]
    with open(p, "wb") as f:
        f.write(struct.pack("<IIII", 0x4151484B, H_q, 1, 256))
        for r in recs:
            f.write(struct.pack("<I", r.shape[1]))
            f.write(r.tobytes())
    hq, hkv, d, got = dump.read_attn_dump(str(p))
    assert (hq, hkv, d, len(got)) == (3, 1, 256, 4)
    m = dump.attn_matrix(str(p))
    assert m.shape == (3, 4, 4)
    np.testing.assert_allclose(m.sum(-1), 1.0, rtol=1e-3)
    assert np.all(np.triu(m[0], 1) == 0)  # causal rows, zeros after n_valid


def test_half_bits_ref_normal_is_round_to_nearest_even():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-9, 9, 100000))).astype(np.float32)
    x = x[np.abs(x) >= 2.0 ** -14]  # normal fp16 results
    x = x[np.abs(x) < 65504]
    np.testing.assert_array_equal(dump.half_bits_ref(x), x.astype(np.float16).view(np.uint16))
    # exact ties round to even
    t = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32)
    assert list(dump.half_bits_ref(t)) == [0x3C00, 0x3C02]


def test_half_bits_ref_subnormal_rounds_half_up():
    # subnormal fp16 results: q = v / 2^-24 rounded half up (ties differ from RNE)
    q = np.array([1.0, 1.5, 2.5, 3.25, 100.5, 1000.0, 1023.4], np.float64)
    v = (q * 2.0 ** -24).astype(np.float32)
    want = np.floor(q + 0.5).astype(np.uint16)
    np.testing.assert_array_equal(dump.half_bits_ref(v), want)
    assert dump.half_bits_ref(np.float32(2.0 ** -25))[()] == 0  # exponent below -9: 0
    assert dump.half_bits_ref(np.float32(2.0 ** -30))[()] == 0
    assert dump.half_bits_ref(np.float32(-7e4))[()] == 0xFC00  # overflow: -inf
