"""GPU parity of the chunked-prefill path: khq_decompress_fp16 against the
float64 decoders (tests/npref.py, pinned to the oracle on the CPU),
khq_prefill_attn_fp16 against float64 causal attention, khq_layer_prefill
against the same tokens stepped one by one, and the C5 configuration (128
queries at positions 8192..8319 with a compression event at the last one)
against the oracle's sequential steps.

Bars: decoded K / V within fp16 rounding (2^-10 of the row block's largest
magnitude); attention outputs within max-abs 2e-3 and rel 1e-3.
"""
import numpy as np
import pytest
import torch

import npref
import oracle
from khq import layer as KL
from khq import ops
from khqdata import (D, H_KV, H_Q, N_REP, SCALE, THETA, layer_consts, random_rows_np,
                     rope_fp16_rows, two_region_state)
from test_gpu_layer import _hip_d2d
from test_gpu_parity import close, payload_from_rows, t

pytestmark = pytest.mark.gpu


def _decoded(rows, h, lc, tok0, n_tok):
    r = {k: v[tok0 * H_KV:(tok0 + n_tok) * H_KV] for k, v in rows.items()}
    K = npref.decode_k(r["kmask"], r["kpay"], r["knorm"], r["krn"], h["cents_k"], h["rotor_k"],
                       h["d_k"], lc.alpha_k).reshape(n_tok, H_KV, D)
    K = npref.rope(K, np.arange(tok0, tok0 + n_tok), THETA)
    V = npref.decode_v(r["vpay"], r["vnorm"], r["vrn"], r["vsm"], h["cents_v"], h["rotor_v"],
                       h["d_v"], h["vq"], lc.alpha_v).reshape(n_tok, H_KV, D)
    return K, V


@pytest.mark.parametrize("data", ["compressed", "random", "outlier-cap"])
def test_decompress_matches_float64_decoders(device, data):
    if data == "compressed":
        st = two_region_state(seed=41, n_tokens=512, boundary=384)
        rows, lc, h = st["rows"], st["lc"], st["h"]
    else:
        lc, h = layer_consts(layer_id=2)
        rows = random_rows_np(384 * H_KV, seed=42)
        if data == "outlier-cap":  # every dim an outlier on some rows: ordinals >= 50
            rows["kmask"][5::7] = 0xFFFFFFFF
    tok0, n_tok, key0 = 21, 301, 40
    pay = payload_from_rows(rows, rows["kmask"].shape[0])
    cents = ops.Centroids(lc, device)
    ld = ops.vt_ld(key0 + n_tok)
    k = torch.zeros(((key0 + n_tok) * H_KV * D,), device=device, dtype=torch.float16)
    vt = torch.zeros((H_KV * D * ld,), device=device, dtype=torch.float16)
    ops.decompress(pay, cents, k, vt, H_kv=H_KV, tok0=tok0, n_tok=n_tok, key0=key0, ld_vt=ld)
    torch.cuda.synchronize()
    K, V = _decoded(rows, h, lc, tok0, n_tok)
    gk = k.cpu().numpy().astype(np.float64).reshape(-1, H_KV, D)[key0:key0 + n_tok]
    gv = vt.cpu().numpy().astype(np.float64).reshape(H_KV, D, ld)[:, :, key0:key0 + n_tok]
    gv = gv.transpose(2, 0, 1)
    assert np.abs(gk - K).max() <= np.abs(K).max() * 2.0 ** -10
    assert np.abs(gv - V).max() <= np.abs(V).max() * 2.0 ** -10
    # roped K against the oracle's own decode through a one-query attention:
    # the decoded rows give the oracle's scores (checked by the attention test
    # below on dense keys); here the rotation itself: |roped| = |unroped|
    assert np.allclose(np.linalg.norm(gk, axis=2), np.linalg.norm(K, axis=2), rtol=2e-3)


def _dense_reference(q_gate, K, V, vis0, n_k):
    n_q = q_gate.shape[0]
    out = np.zeros((n_q, H_Q, D))
    qf = q_gate.astype(np.float64)
    for j in range(n_q):
        vis = min(n_k, vis0 + j)
        for hq in range(H_Q):
            kv = hq // N_REP
            s = K[:vis, kv, :] @ qf[j, hq, :D] * SCALE
            p = np.exp(s - s.max())
            o = (p @ V[:vis, kv, :]) / (p.sum() + 1e-8)
            out[j, hq] = o / (1.0 + np.exp(-qf[j, hq, D:]))
    return out


@pytest.mark.parametrize("n_k,n_q,vis0", [(300, 37, 264), (1000, 128, 873), (16, 1, 1),
                                           (77, 5, 70)])
def test_prefill_attn_vs_float64(device, n_k, n_q, vis0):
    rng = np.random.default_rng(n_k + n_q)
    K = rng.standard_normal((n_k, H_KV, D)).astype(np.float16)
    V = rng.standard_normal((n_k, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((n_q, H_Q, 2 * D)).astype(np.float16)
    ld = ops.vt_ld(n_k)
    vt = np.zeros((H_KV, D, ld), np.float16)
    vt[:, :, :n_k] = V.transpose(1, 2, 0)
    vt[:, :, n_k:] = np.float16(np.nan)  # padding must never be read as values
    out = torch.zeros((n_q, H_Q, D), device=device, dtype=torch.float16)
    ops.prefill_attn(t(q), t(K), t(vt), out, ld_vt=ld, n_k=n_k, n_q=n_q, vis0=vis0, H_q=H_Q,
                     H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    want = _dense_reference(q, K.astype(np.float64), V.astype(np.float64), vis0, n_k)
    close(out.cpu().numpy(), want)


@pytest.mark.parametrize("n_k,n_q,vis0", [(333, 37, 297), (44, 3, 40), (1000 - 24, 130, 847)])
def test_prefill_attn_minimum_vt_leading_dim(device, n_k, n_q, vis0):
    """n_k % 32 in 1..16 with ld_vt at its minimum (n_k rounded up to 32) and a
    V^T buffer of exactly H_kv * 256 * ld_vt halves: the last 32-key tile of
    the last head ends at the buffer's end."""
    rng = np.random.default_rng(n_k * 7 + n_q)
    K = rng.standard_normal((n_k, H_KV, D)).astype(np.float16)
    V = rng.standard_normal((n_k, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((n_q, H_Q, 2 * D)).astype(np.float16)
    ld = (n_k + 31) // 32 * 32
    assert 1 <= n_k % 32 <= 16
    vt = np.zeros((H_KV, D, ld), np.float16)
    vt[:, :, :n_k] = V.transpose(1, 2, 0)
    out = torch.zeros((n_q, H_Q, D), device=device, dtype=torch.float16)
    ops.prefill_attn(t(q), t(K), t(vt), out, ld_vt=ld, n_k=n_k, n_q=n_q, vis0=vis0, H_q=H_Q,
                     H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    want = _dense_reference(q, K.astype(np.float64), V.astype(np.float64), vis0, n_k)
    close(out.cpu().numpy(), want)


def _tokens(n, seed, pos0=0):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n, H_KV, D)).astype(np.float16)
    v = rng.standard_normal((n, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((n, H_Q, 2 * D)).astype(np.float16)
    return k, rope_fp16_rows(k, np.arange(pos0, pos0 + n)), v, q


def _payload_np(layer, n_tok):
    ptrs = layer.payload_ptrs()
    n = n_tok * H_KV
    shapes = [("kmask", (n, 16), torch.int32), ("kpay", (n, 40), torch.uint8),
              ("knorm", (n,), torch.float16), ("krn", (n,), torch.float16),
              ("vpay", (n, 104), torch.uint8), ("vnorm", (n,), torch.float16),
              ("vrn", (n,), torch.float16), ("vsm", (n, 4), torch.uint8)]
    out = {}
    torch.cuda.synchronize()
    for i, (name, shape, dt) in enumerate(shapes):
        buf = torch.empty(shape, device="cuda", dtype=dt)
        assert _hip_d2d(buf.data_ptr(), ptrs[i], buf.numel() * buf.element_size()) == 0
        out[name] = buf.cpu().numpy()
    out["kmask"] = out["kmask"].view(np.uint32)
    rings = []
    for i in (8, 9):
        buf = torch.empty((256, H_KV, D), device="cuda", dtype=torch.float16)
        assert _hip_d2d(buf.data_ptr(), ptrs[i], buf.numel() * 2) == 0
        rings.append(buf.cpu().numpy())
    return out, rings


def test_layer_prefill_matches_steps(device):
    """Chunks of several sizes (one that must be cut where its ring writes
    would overwrite slots still read) against the same tokens stepped: same
    cadence and compressed bytes, outputs within tolerance (the prefill
    attends over fp16-decoded keys)."""
    lc, _ = layer_consts(layer_id=7)
    opt = KL.KhqOptions(splits=8, fused=True)
    st = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    pf = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    n = 700
    k, kr, v, q = _tokens(n, seed=19)
    o_step = torch.empty((n, H_Q, D), device=device, dtype=torch.float16)
    for i in range(n):
        assert st.step(t(q[i]), t(kr[i]), t(v[i]), o_step[i], SCALE, k_unroped=t(k[i]))
    o_pf = torch.empty_like(o_step)
    i = 0
    for m in (1, 5, 250, 128, 100, 216):
        assert pf.prefill(t(q[i:i + m]), t(kr[i:i + m]), t(v[i:i + m]), t(k[i:i + m]),
                          o_pf[i:i + m], SCALE) == m
        i += m
    assert i == n
    torch.cuda.synchronize()
    assert pf.state() == st.state() == (512, 700, 4)
    a, ra = _payload_np(st, 512)
    b, rb = _payload_np(pf, 512)
    for name in a:
        assert np.array_equal(a[name], b[name]), name
    assert np.array_equal(ra[0], rb[0]) and np.array_equal(ra[1], rb[1])
    got, want = o_pf.cpu().numpy(), o_step.cpu().numpy()
    for j in range(n):  # every query: the runs before and after each event
        close(got[j], want[j])


@pytest.mark.parametrize("H_q,H_kv,n_q,n_k", [(8, 2, 50, 520), (12, 1, 9, 200), (4, 4, 3, 97)])
def test_prefill_attn_other_gqa_shapes_vs_float64(device, H_q, H_kv, n_q, n_k):
    """Other GQA shapes through khq_prefill_attn_fp16 (rows = n_q x n_rep of
    each KV head: 200 and 108 rows take the role-specialised 32-row kernel
    and the 16-row kernel respectively) against float64 causal attention."""
    rep = H_q // H_kv
    rng = np.random.default_rng(H_q * 100 + n_q)
    K = rng.standard_normal((n_k, H_kv, D)).astype(np.float16)
    V = rng.standard_normal((n_k, H_kv, D)).astype(np.float16)
    q = rng.standard_normal((n_q, H_q, 2 * D)).astype(np.float16)
    vis0 = n_k - n_q + 1
    ld = ops.vt_ld(n_k)
    vt = np.zeros((H_kv, D, ld), np.float16)
    vt[:, :, :n_k] = V.transpose(1, 2, 0)
    out = torch.zeros((n_q, H_q, D), device=device, dtype=torch.float16)
    ops.prefill_attn(t(q), t(K), t(vt), out, ld_vt=ld, n_k=n_k, n_q=n_q, vis0=vis0, H_q=H_q,
                     H_kv=H_kv, scale=SCALE)
    torch.cuda.synchronize()
    qf, Kd, Vd = q.astype(np.float64), K.astype(np.float64), V.astype(np.float64)
    want = np.zeros((n_q, H_q, D))
    for j in range(n_q):
        vis = min(n_k, vis0 + j)
        for hq in range(H_q):
            kv = hq // rep
            sc = Kd[:vis, kv, :] @ qf[j, hq, :D] * SCALE
            p = np.exp(sc - sc.max())
            want[j, hq] = (p @ Vd[:vis, kv, :]) / (p.sum() + 1e-8) / (1.0 + np.exp(-qf[j, hq, D:]))
    close(out.cpu().numpy(), want)


def test_prefill_attn_rescales_vs_float64(device):
    """Keys whose magnitude ramps up along the sequence: the row maxima rise by
    more than the lazy-rescale gap several times within a split, so the
    output side applies the rescale factors the score side hands over (the
    32-row role-specialised kernel: 40 queries x 6 heads = 240 rows)."""
    n_k, n_q, vis0 = 640, 40, 601
    rng = np.random.default_rng(61)
    ramp = (1.0 + np.arange(n_k) / 24.0).astype(np.float32)[:, None, None]
    K = (rng.standard_normal((n_k, H_KV, D)) * 0.5 * ramp).astype(np.float16)
    V = rng.standard_normal((n_k, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((n_q, H_Q, 2 * D)).astype(np.float16)
    ld = ops.vt_ld(n_k)
    vt = np.zeros((H_KV, D, ld), np.float16)
    vt[:, :, :n_k] = V.transpose(1, 2, 0)
    out = torch.zeros((n_q, H_Q, D), device=device, dtype=torch.float16)
    ops.prefill_attn(t(q), t(K), t(vt), out, ld_vt=ld, n_k=n_k, n_q=n_q, vis0=vis0, H_q=H_Q,
                     H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    Kd = K.astype(np.float64)
    want = _dense_reference(q, Kd, V.astype(np.float64), vis0, n_k)
    # the test is meaningful only if the maxima rise by more than the gap
    s_first = Kd[:32, 0, :] @ q[0, 0, :D].astype(np.float64) * SCALE
    s_all = Kd[:vis0, 0, :] @ q[0, 0, :D].astype(np.float64) * SCALE
    assert s_all.max() - s_first.max() > 10.0
    close(out.cpu().numpy(), want)


@pytest.mark.parametrize("chunks", [(128,) * 6, (1, 5, 250, 128, 100, 216)])
def test_layer_prefill_decoded_rows_match_decode(device, chunks):
    """The dense key space a layer's prefills build (compression events that
    decode their own rows in the compressing launch, with the chunk append
    beside them) holds, bit for bit, what khq_decompress_fp16 makes of the
    layer's compressed rows."""
    lc, _ = layer_consts(layer_id=5)
    L = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device,
                          options=KL.KhqOptions(splits=8, fused=True))
    n = sum(chunks)
    k, kr, v, q = _tokens(n, seed=37)
    out = torch.empty((n, H_Q, D), device=device, dtype=torch.float16)
    i = 0
    for m in chunks:
        assert L.prefill(t(q[i:i + m]), t(kr[i:i + m]), t(v[i:i + m]), t(k[i:i + m]),
                         out[i:i + m], SCALE) == m
        i += m
    torch.cuda.synchronize()
    boundary = L.state()[0]
    kp, vtp, ld, n_dec = L.dense()
    assert 384 <= n_dec <= boundary
    got_k = torch.empty((n_dec * H_KV * D,), device=device, dtype=torch.float16)
    assert _hip_d2d(got_k.data_ptr(), kp, got_k.numel() * 2) == 0
    got_vt = torch.empty((H_KV * D * ld,), device=device, dtype=torch.float16)
    assert _hip_d2d(got_vt.data_ptr(), vtp, got_vt.numel() * 2) == 0
    rows, _ = _payload_np(L, n_dec)
    pay = payload_from_rows(rows, n_dec * H_KV)
    ld2 = ops.vt_ld(n_dec)
    want_k = torch.zeros((n_dec * H_KV * D,), device=device, dtype=torch.float16)
    want_vt = torch.zeros((H_KV * D * ld2,), device=device, dtype=torch.float16)
    ops.decompress(pay, ops.Centroids(lc, device), want_k, want_vt, H_kv=H_KV, tok0=0,
                   n_tok=n_dec, key0=0, ld_vt=ld2)
    torch.cuda.synchronize()
    gk = got_k.cpu().numpy().view(np.uint16)
    wk = want_k.cpu().numpy().view(np.uint16)
    assert np.array_equal(gk, wk)
    gv = got_vt.cpu().numpy().view(np.uint16).reshape(H_KV * D, ld)[:, :n_dec]
    wv = want_vt.cpu().numpy().view(np.uint16).reshape(H_KV * D, ld2)[:, :n_dec]
    assert np.array_equal(gv, wv)


def test_c5_chunk_vs_oracle(device):
    """Config 5: 8,192 tokens already appended (boundary 8,064, raw 8,064..
    8,191), then one chunk of 128 tokens at positions 8,192..8,319; the 128th
    append compresses 8,064..8,191.  Queries 0, 1, 63, 126 see c_len 8,064 and
    129 + j raw tokens, query 127 sees c_len 8,192 and 128 raw tokens."""
    lc, h = layer_consts(layer_id=4)
    L = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=8448, device=device,
                          options=KL.KhqOptions(splits=16, fused=True))
    n0 = 8192
    k, kr, v, q = _tokens(n0 + 128, seed=23)
    scratch = torch.empty((128, H_Q, D), device=device, dtype=torch.float16)
    for i in range(0, n0, 128):
        L.prefill(t(q[i:i + 128]), t(kr[i:i + 128]), t(v[i:i + 128]), t(k[i:i + 128]), scratch,
                  SCALE)
    assert L.state() == (8064, 8192, 63)
    out = torch.empty((128, H_Q, D), device=device, dtype=torch.float16)
    L.prefill(t(q[n0:]), t(kr[n0:]), t(v[n0:]), t(k[n0:]), out, SCALE)
    torch.cuda.synchronize()
    assert L.state() == (8192, 8320, 64)
    rows, (ring_k, ring_v) = _payload_np(L, 8192)
    got = out.cpu().numpy()
    for j in (0, 1, 63, 126, 127):
        c_len = 8064 if j < 127 else 8192
        win_start, win_len = c_len % 256, n0 + j + 1 - c_len
        qj = np.ascontiguousarray(q[n0 + j])
        _, ac, _ = oracle.attn(qj, rows["kpay"], rows["vpay"], rows["vsm"], rows["kmask"],
                               rows["knorm"], rows["krn"], rows["vnorm"], rows["vrn"],
                               h["cents_k"], h["cents_v"], h["vq"], h["rotor_k"], h["rotor_v"],
                               h["d_k"], h["d_v"], num_queries=H_Q, num_heads=H_Q, L_q=1,
                               c_len=c_len, n_rep=N_REP, scale=SCALE, alpha_k=lc.alpha_k,
                               alpha_v=lc.alpha_v, rope_base=THETA, start_pos=0, num_splits=16)
        _, aw = oracle.window_attn(qj, ring_k, ring_v, win_start=win_start, win_len=win_len,
                                   ring_cap=256, H_q=H_Q, H_kv=H_KV, scale=SCALE)
        _, want = oracle.merge_gate(ac, aw, qj, H_q=H_Q, has_w=True)
        close(got[j], want)


def test_layer_prefill_mixed_with_steps(device):
    """Prefill chunks and single steps interleaved on one layer (the dense key
    space must not keep raw tokens the steps wrote only to the ring) against
    the same tokens stepped one by one."""
    lc, _ = layer_consts(layer_id=9)
    opt = KL.KhqOptions(splits=8, fused=True)
    st = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    mx = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    n = 420
    k, kr, v, q = _tokens(n, seed=29)
    o_step = torch.empty((n, H_Q, D), device=device, dtype=torch.float16)
    for i in range(n):
        assert st.step(t(q[i]), t(kr[i]), t(v[i]), o_step[i], SCALE, k_unroped=t(k[i]))
    o_mx = torch.empty_like(o_step)
    i = 0
    for kind, m in (("p", 100), ("s", 3), ("p", 60), ("s", 1), ("p", 97), ("s", 30), ("p", 129)):
        if kind == "p":
            assert mx.prefill(t(q[i:i + m]), t(kr[i:i + m]), t(v[i:i + m]), t(k[i:i + m]),
                              o_mx[i:i + m], SCALE) == m
        else:
            for j in range(i, i + m):
                assert mx.step(t(q[j]), t(kr[j]), t(v[j]), o_mx[j], SCALE, k_unroped=t(k[j]))
        i += m
    assert i == n
    torch.cuda.synchronize()
    assert mx.state() == st.state()
    got, want = o_mx.cpu().numpy(), o_step.cpu().numpy()
    for j in list(range(0, n, 7)) + [99, 100, 102, 103, 162, 163, 164, 260, 290, 291, n - 1]:
        close(got[j], want[j])
