"""The native dump recorder (khq_dump_*) on the GPU: KHQD rows equal the
appended K/V, KHQA scores equal a float64 softmax of q.k over the layer's
roped-K history within one fp16 ulp (written with the reference's rounding,
ref:src/models/qwen3_5/khq_dump.mojo:199-316), limits and resets."""
import numpy as np
import pytest
import torch

from khq import dump

pytestmark = pytest.mark.gpu

H_Q, H_KV, D = 24, 4, 256
KV = H_KV * D


def _want_scores(qs, ks, pos, scale):
    """float64 softmax of token pos (q row per head) over keys 0..pos."""
    q = qs[pos].astype(np.float64)[:, :D]                 # [H_q, D]
    k = ks[:pos + 1].astype(np.float64).reshape(pos + 1, H_KV, D)
    n_rep = H_Q // H_KV
    out = np.zeros((H_Q, pos + 1))
    for h in range(H_Q):
        s = k[:, h // n_rep, :] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = p / p.sum()
    return out


def test_recorder_kv_and_attn(device, tmp_path):
    rng = np.random.default_rng(0)
    T, cap, scale = 40, 32, 1.0 / 16.0
    rec = dump.Recorder(str(tmp_path), max_tokens=cap, kv_dim=KV)
    ks = rng.standard_normal((T, KV)).astype(np.float16)
    vs = rng.standard_normal((T, KV)).astype(np.float16)
    kr = (rng.standard_normal((T, KV)) * 0.5).astype(np.float16)
    qs = (rng.standard_normal((T, H_Q, 2 * D)) * 0.5).astype(np.float16)
    for pos in range(T):
        print(f"dump token {pos}", flush=True)
        for layer in (5, 2):
            rec.kv(layer, torch.from_numpy(ks[pos]).to(device), torch.from_numpy(vs[pos]).to(device))
            rec.attn(layer, torch.from_numpy(qs[pos]).to(device), torch.from_numpy(kr[pos]).to(device),
                     pos, H_q=H_Q, H_kv=H_KV, D=D, scale=scale)
    assert rec.count(5) == cap and rec.count(2) == cap  # capped at max_tokens
    rec.flush()
    kvd = dump.read_kv_dump(str(tmp_path / "kv_dump.bin"))
    assert list(kvd) == [2, 5]  # layer-id order
    for layer in (2, 5):
        np.testing.assert_array_equal(kvd[layer][0], ks[:cap].astype(np.float32))
        np.testing.assert_array_equal(kvd[layer][1], vs[:cap].astype(np.float32))
    for layer in (2, 5):
        hq, hkv, d, recs = dump.read_attn_dump(str(tmp_path / f"attn_{layer}.bin"))
        assert (hq, hkv, d, len(recs)) == (H_Q, H_KV, D, cap)  # pos >= cap not recorded
        for pos in (0, 1, 7, cap - 1):
            want = dump.half_bits_ref(_want_scores(qs, kr, pos, scale).astype(np.float32))
            got = recs[pos].view(np.uint16)
            assert got.shape == (H_Q, pos + 1)
            assert np.abs(got.astype(np.int32) - want.astype(np.int32)).max() <= 1
    rec.close()


def test_recorder_new_sequence_and_shape_guard(device, tmp_path):
    rng = np.random.default_rng(1)
    rec = dump.Recorder(str(tmp_path), max_tokens=16, kv_dim=KV, flags=dump.DUMP_ATTN)
    kr = (rng.standard_normal((6, KV)) * 0.5).astype(np.float16)
    qs = (rng.standard_normal((6, H_Q, 2 * D)) * 0.5).astype(np.float16)
    for pos in range(3):
        rec.attn(0, torch.from_numpy(qs[pos]).to(device), torch.from_numpy(kr[pos]).to(device),
                 pos, H_q=H_Q, H_kv=H_KV, D=D, scale=0.0625)
    # pos 0 again: a new sequence, the history restarts
    for pos in range(2):
        rec.attn(0, torch.from_numpy(qs[3 + pos]).to(device),
                 torch.from_numpy(kr[3 + pos]).to(device), pos, H_q=H_Q, H_kv=H_KV, D=D,
                 scale=0.0625)
    # a different head count than the first call is ignored
    rec.attn(0, torch.from_numpy(qs[0, :12]).to(device), torch.from_numpy(kr[0]).to(device), 2,
             H_q=12, H_kv=H_KV, D=D, scale=0.0625)
    rec.flush()
    _, _, _, recs = dump.read_attn_dump(str(tmp_path / "attn_0.bin"))
    assert [r.shape[1] for r in recs] == [1, 2, 3, 1, 2]
    want = dump.half_bits_ref(_want_scores(qs[3:], kr[3:], 1, 0.0625).astype(np.float32))
    assert np.abs(recs[4].view(np.uint16).astype(np.int32) - want.astype(np.int32)).max() <= 1
    assert not (tmp_path / "kv_dump.bin").exists()  # KHQD not enabled
    rec.close()
