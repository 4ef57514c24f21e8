"""khq_layer_attention_step (ref:src/models/qwen3_5/attention.mojo:319-365):
head RMSNorm -> unroped capture -> partial RoPE -> KHQ step, through the C ABI.

The front is checked against a float64 RMSNorm (the closed form of
ref:src/models/qwen3_5/norm.mojo:72-85 / elementwise_sm75.mojo:362-423,
weight applied after the scale, fp16 stored) and the oracle's
partial_rope_fp16 on those fp16 values; the step is checked bit for bit
against khq_layer_step fed with the tensors the front produced, over enough
tokens for three compression events; the dump hooks record the normed
pre-RoPE K and V and one score record per token."""
import numpy as np
import pytest
import torch

import oracle
from khq import dump
from khq.centroids import synthetic_layer
from khq.layer import ROPE_BASE, KhqOptions, NativeKhqLayer

pytestmark = pytest.mark.gpu

H_Q, H_KV, D = 24, 4, 256
SCALE = 1.0 / 16.0
EPS = 1e-6


def _d2d(dst, src, nbytes, kind=3):
    from test_gpu_layer import _hip_d2d

    assert _hip_d2d(dst, src, nbytes) == 0


def rmsnorm64(x, heads, stride, w):
    """float64 head RMSNorm of the first 256 values of each head row, fp16 out."""
    x = np.asarray(x, np.float16).astype(np.float64).reshape(heads, stride)[:, :D]
    inv = 1.0 / np.sqrt((x ** 2).sum(1, keepdims=True) / D + EPS)
    y = x * inv
    if w is not None:
        y = y * w.astype(np.float64)[None, :]
    return y.astype(np.float16)


def ulps16(a, b):
    a = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    b = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    a = np.where(a < 0, -32768 - a, a)
    b = np.where(b < 0, -32768 - b, b)
    return np.abs(a - b)


def _layers(opt):
    lc = synthetic_layer(3, seed=1234)
    return (NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, options=opt),
            NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, options=opt))


@pytest.mark.parametrize("weights", [False, True])
def test_front_matches_float64_norm_and_oracle_rope(device, weights):
    rng = np.random.default_rng(7)
    A, _ = _layers(KhqOptions(splits=16, fused=True))
    qw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(device) if weights else None
    kw = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).to(device) if weights else None
    out = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    for pos in range(5):
        q = (rng.standard_normal((H_Q, 2 * D)) * 3).astype(np.float16)
        k = (rng.standard_normal((H_KV, D)) * 3).astype(np.float16)
        v = rng.standard_normal((H_KV, D)).astype(np.float16)
        qt, kt, vt = (torch.from_numpy(a).to(device) for a in (q, k, v))
        A.attention_step(qt, kt, vt, out, SCALE, pos=pos, q_norm_w=qw, k_norm_w=kw, eps=EPS)
        torch.cuda.synchronize()
        qn = rmsnorm64(q, H_Q, 2 * D, qw.cpu().numpy() if weights else None)
        kn = rmsnorm64(k, H_KV, D, kw.cpu().numpy() if weights else None)
        ptrs = A.payload_ptrs()
        slot = pos % 256
        ring = {}
        for name, idx in (("k", 8), ("v", 9), ("u", 10)):
            t = torch.empty((H_KV, D), device=device, dtype=torch.float16)
            nb = H_KV * D * 2
            _d2d(t.data_ptr(), ptrs[idx] + slot * nb, nb)
            ring[name] = t.cpu().numpy()
        # normed pre-RoPE K in ring_u, within one fp16 ulp of float64
        assert ulps16(ring["u"], kn).max() <= 1
        np.testing.assert_array_equal(ring["v"], v)
        # RoPE of the stored normed values: the oracle's partial_rope on them
        want_k = oracle.partial_rope_fp16(ring["u"], num_heads=H_KV, head_dim=D, rotary_dim=64,
                                          pos=pos, theta=ROPE_BASE)
        got_k = kt.cpu().numpy()
        assert ulps16(got_k, want_k).max() <= 1
        np.testing.assert_array_equal(ring["k"], got_k)
        got_q = qt.cpu().numpy()
        assert ulps16(got_q[:, 64:D], qn[:, 64:]).max() <= 1  # dims past the rotary part
        want_q = oracle.partial_rope_fp16(np.concatenate([qn, q[:, D:]], 1), num_heads=H_Q,
                                          head_dim=D, rotary_dim=64, pos=pos, theta=ROPE_BASE,
                                          stride=2 * D)
        assert ulps16(got_q[:, :64], want_q[:, :64]).max() <= 2
        np.testing.assert_array_equal(got_q[:, D:], q[:, D:])  # the gate half is untouched


def test_step_matches_layer_step_over_three_events(device):
    """attention_step == khq_layer_step on the front's own outputs, bit for bit,
    over 520 tokens (compression events at 256, 384, 512)."""
    rng = np.random.default_rng(8)
    A, B = _layers(KhqOptions(splits=16, fused=True))
    outA = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    outB = torch.empty_like(outA)
    ku = torch.empty((H_KV, D), device=device, dtype=torch.float16)
    for pos in range(520):
        q = torch.from_numpy((rng.standard_normal((H_Q, 2 * D)) * 2).astype(np.float16)).to(device)
        k = torch.from_numpy((rng.standard_normal((H_KV, D)) * 2).astype(np.float16)).to(device)
        v = torch.from_numpy(rng.standard_normal((H_KV, D)).astype(np.float16)).to(device)
        okA = A.attention_step(q, k, v, outA, SCALE, pos=pos, eps=EPS)
        ptrs = A.payload_ptrs()
        nb = H_KV * D * 2
        _d2d(ku.data_ptr(), ptrs[10] + (pos % 256) * nb, nb)
        okB = B.step(q, k, v, outB, SCALE, k_unroped=ku)  # q, k: normed and roped now
        assert okA == okB
        if pos in (0, 255, 256, 300, 383, 384, 511, 512, 519):
            torch.cuda.synchronize()
            print(f"attention_step pos {pos}", flush=True)
            assert torch.equal(outA, outB)
            assert A.state() == B.state()
    assert A.state() == (384, 520, 3)  # cadence: events at 256, 384, 512


def test_dump_hooks(device, tmp_path):
    rng = np.random.default_rng(9)
    A, _ = _layers(KhqOptions(splits=16, fused=True))
    rec = dump.Recorder(str(tmp_path), max_tokens=64, kv_dim=H_KV * D)
    A.set_dump(rec, layer_id=3)
    out = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    ks, vs = [], []
    for pos in range(12):
        q = torch.from_numpy(rng.standard_normal((H_Q, 2 * D)).astype(np.float16)).to(device)
        k = torch.from_numpy(rng.standard_normal((H_KV, D)).astype(np.float16)).to(device)
        v = torch.from_numpy(rng.standard_normal((H_KV, D)).astype(np.float16)).to(device)
        A.attention_step(q, k, v, out, SCALE, pos=pos, eps=EPS)
        ptrs = A.payload_ptrs()
        u = torch.empty((H_KV, D), device=device, dtype=torch.float16)
        _d2d(u.data_ptr(), ptrs[10] + pos * H_KV * D * 2, H_KV * D * 2)
        ks.append(u.cpu().numpy().reshape(-1))
        vs.append(v.cpu().numpy().reshape(-1))
    A.set_dump(None, 0)
    rec.flush()
    kvd = dump.read_kv_dump(str(tmp_path / "kv_dump.bin"))
    np.testing.assert_array_equal(kvd[3][0], np.stack(ks).astype(np.float32))
    np.testing.assert_array_equal(kvd[3][1], np.stack(vs).astype(np.float32))
    _, _, _, recs = dump.read_attn_dump(str(tmp_path / "attn_3.bin"))
    assert [r.shape for r in recs] == [(H_Q, p + 1) for p in range(12)]
    for r in recs:
        np.testing.assert_allclose(r.astype(np.float64).sum(1), 1.0, atol=2e-2)
    rec.close()
