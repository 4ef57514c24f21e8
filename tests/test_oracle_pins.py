"""Pins the C oracle (CPU, no GPU needed).

The reference ships no KHQ unit test or golden vector, so each oracle
function is checked against something it cannot agree with by accident:
an independent float64 numpy decoder + brute-force attention (tests/npref.py),
closed forms (H.H = 256 I, orthogonal rotors, logsumexp merge of any
partition), brute force on small inputs (exhaustive codeword search) and the
reference's own GQA / RoPE test cases.
"""
import numpy as np
import pytest

import npref
import oracle
from khqdata import (D, H_KV, H_Q, N_REP, SCALE, THETA, compress_rows, layer_consts,
                     oracle_attn, oracle_window, random_rows_np, rope_fp16_rows,
                     stressed_rows_np, two_region_state)


def cos_sim(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


# ------------------------------------------------------------------ compress
def _proj64(x, d, rotor):
    """float64 projection: rot = R^T (H (x*d/|x|)) / 16 per patch."""
    x = np.asarray(x, np.float64)
    r = x * npref.f16(d)[None, :] / np.linalg.norm(x, axis=1, keepdims=True)
    r = r @ npref.H256.T
    R = npref.f16(rotor).reshape(64, 4, 4)  # rotor[p][k][c]
    return np.einsum("pkc,npk->npc", R, r.reshape(-1, 64, 4)).reshape(-1, D) / 16.0


def test_compress_k_roundtrip_and_codes():
    lc, h = layer_consts()
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 1, D)).astype(np.float16)
    kmask, knorm, krn, kpay, sm = compress_rows(x, h, False)
    # norm: fp16 of sqrt(sum x^2)
    xn = np.linalg.norm(x.reshape(64, D).astype(np.float64), axis=1)
    np.testing.assert_allclose(knorm.astype(np.float64), xn, rtol=1e-3)
    assert np.all(sm.view(np.uint32) == 0)
    assert np.all(kpay[:, 36] == 2) and np.all(kpay[:, 37:] == 0)
    # decoded K is alpha_k * x / 16 (the reference's K scale) up to 2-bit loss
    kdec = npref.decode_k(kmask, kpay, knorm, krn, h["cents_k"], h["rotor_k"], h["d_k"],
                          lc.alpha_k)
    for i in range(64):
        assert cos_sim(kdec[i], x[i, 0]) > 0.9
    ratio = np.linalg.norm(kdec, axis=1) / (xn / 16.0)
    assert np.all((ratio > 0.7) & (ratio < 1.3))
    # codes against float64 thresholds, away from the decision boundaries
    proj = _proj64(x.reshape(64, D), h["d_k"], h["rotor_k"])
    f_s = 1.0 / 16.0
    codes = (kmask[:, np.arange(D) // 16] >> (2 * (np.arange(D) % 16)).astype(np.uint32)) & 3
    a = np.abs(proj)
    safe = (np.abs(a - 1.6 * f_s) > 1e-5) & (np.abs(a - 0.47 * f_s) > 1e-5)
    cand = a > 1.6 * f_s
    ordn = np.cumsum(cand, 1) - cand
    want = np.where(proj > 0.47 * f_s, 2, np.where(proj < -0.47 * f_s, 1, 0))
    want = np.where(cand, np.where(ordn < 50, 3, np.where(proj > 0, 2, 1)), want)
    rows_safe = safe.all(1)
    assert rows_safe.sum() > 32
    assert np.array_equal(codes[rows_safe], want[rows_safe])
    # outlier signs are the signs of proj (bit j of bytes 29..35, 1 = positive)
    for i in np.nonzero(rows_safe)[0][:8]:
        dims = np.nonzero(codes[i] == 3)[0]
        bits = [(kpay[i, 29 + j // 8] >> (j % 8)) & 1 for j in range(len(dims))]
        assert bits == [int(proj[i, d] > 0) for d in dims]


def test_compress_k_outlier_cap_50():
    lc, h = layer_consts()
    rng = np.random.default_rng(1)
    # rows built from a target projection with 40..120 dims far above the
    # outlier threshold (x = d * H (R p) / 16, inverting the compress transform)
    tgt = rng.standard_normal((16, D)) * 0.3
    for i in range(16):
        n_big = 40 + 5 * i
        idx = rng.choice(D, n_big, replace=False)
        tgt[i, idx] = rng.choice([-2.5, 2.5], n_big)
    R = npref.f16(h["rotor_k"]).reshape(64, 4, 4)  # rotor[p][k][c]: rot = R^T r
    r = np.einsum("pkc,npc->npk", R, tgt.reshape(16, 64, 4)).reshape(16, D)
    x = ((r @ npref.H256.T) * npref.f16(h["d_k"])[None, :] * 4.0).astype(np.float16)[:, None, :]
    kmask, knorm, krn, kpay, _ = compress_rows(x, h, False)
    codes = (kmask[:, np.arange(D) // 16] >> (2 * (np.arange(D) % 16)).astype(np.uint32)) & 3
    n3 = (codes == 3).sum(1)
    assert n3.max() == 50 and n3.min() < 50
    proj = _proj64(x.reshape(16, D), h["d_k"], h["rotor_k"])
    n_cand = (np.abs(proj) > 1.6 / 16).sum(1)
    np.testing.assert_array_equal(n3, np.minimum(n_cand, 50))


def test_compress_zero_row():
    lc, h = layer_consts()
    x = np.zeros((4, 1, D), np.float16)
    kmask, knorm, krn, kpay, _ = compress_rows(x, h, False)
    assert np.all(kmask == 0)
    assert np.all(knorm.astype(np.float32) == np.float32(np.float16(np.sqrt(np.float32(1e-8)))))
    assert np.all(krn == 0)
    assert np.all(kpay[:, 0:4].copy().view(np.uint32) == 1000)  # mult defaults to 1.0


def test_compress_v_roundtrip_and_vq_bruteforce():
    # codebook scale matched to the projection (alpha_v = 1/16)
    lc, h = layer_consts(alpha_v=1.0 / 16.0)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 1, D)).astype(np.float16)
    X = np.ascontiguousarray(x.reshape(32, D))
    rc, _, vnorm, vrn, vpay, vsm = oracle.compress(X, h["d_v"], h["rotor_v"], h["cents_v"],
                                                   h["vq"], ts=1.95, alpha=1.0 / 16.0, is_v=True)
    assert rc == 0
    vdec = npref.decode_v(vpay, vnorm, vrn, vsm, h["cents_v"], h["rotor_v"], h["d_v"], h["vq"],
                          1.0 / 16.0)
    for i in range(32):
        assert cos_sim(vdec[i], X[i]) > 0.85
    # exhaustive codeword search in float64 where the winner is clear
    proj = _proj64(X, h["d_v"], h["rotor_v"]).reshape(32, 64, 4)
    cb = npref.f16(h["vq"]).reshape(64, 256, 3) / 16.0
    dist = ((proj[:, :, None, :3] - cb[None]) ** 2).sum(-1)  # [n, 64, 256]
    order = np.sort(dist, axis=2)
    clear = (order[:, :, 1] - order[:, :, 0]) > 1e-6 * (1 + order[:, :, 0])
    code, d3c, dump = npref.unpack_v_fields(vpay)
    assert clear.mean() > 0.9
    np.testing.assert_array_equal(code[clear], dist.argmin(2)[clear])
    # shared meta = max |dim-3 residual|; dumps within [0, 15]
    sm = vsm.view(np.float32).ravel()
    cv = npref.f16(h["cents_v"]).reshape(4, D)[:, np.arange(64) * 4 + 3] / 16.0
    res = proj[:, :, 3] - cv[d3c, np.arange(64)[None, :]]
    np.testing.assert_allclose(sm, np.abs(res).max(1), rtol=1e-4, atol=1e-7)
    assert dump.min() >= 0 and dump.max() <= 15


def test_vq_tie_takes_first_codeword():
    lc, h = layer_consts(alpha_v=1.0 / 16.0)
    vq = h["vq"].reshape(64, 256, 3).copy()
    vq[:, 200] = vq[:, 10]  # duplicate codeword 10 at 200
    rng = np.random.default_rng(3)
    X = rng.standard_normal((8, D)).astype(np.float16)
    rc, _, _, _, vpay, _ = oracle.compress(X, h["d_v"], h["rotor_v"], h["cents_v"],
                                           vq.reshape(-1), ts=1.95, alpha=1.0 / 16.0, is_v=True)
    code, _, _ = npref.unpack_v_fields(vpay)
    assert not np.any(code == 200)


# ----------------------------------------------------------------- attention
def _brute_compressed(st, c_len, start_pos=0):
    r, h, lc = st["rows"], st["h"], st["lc"]
    K = npref.decode_k(r["kmask"], r["kpay"], r["knorm"], r["krn"], h["cents_k"], h["rotor_k"],
                       h["d_k"], lc.alpha_k).reshape(-1, H_KV, D)[:c_len]
    K = npref.rope(K, np.arange(start_pos, start_pos + c_len), THETA)
    V = npref.decode_v(r["vpay"], r["vnorm"], r["vrn"], r["vsm"], h["cents_v"], h["rotor_v"],
                       h["d_v"], h["vq"], lc.alpha_v).reshape(-1, H_KV, D)[:c_len]
    q = npref.f16(st["q_gate"])[:, :D]
    return K, V, q


@pytest.mark.parametrize("splits", [1, 8])
def test_attn_oracle_vs_bruteforce(splits):
    st = two_region_state(seed=11)
    rc, out, part = oracle_attn(st, num_splits=splits)
    assert rc == 0
    K, V, q = _brute_compressed(st, st["c_len"])
    want, lse = npref.attention(q, K, V, SCALE, N_REP)
    got, glse = npref.triple_to_out(out)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(glse, lse, rtol=1e-5, atol=1e-5)


def test_attn_oracle_random_rows_long_and_reanchor():
    # > 256 tokens per split exercises the RoPE re-anchor at s % 256 == 0
    lc, h = layer_consts()
    rows = random_rows_np(700 * H_KV, seed=5)
    rng = np.random.default_rng(6)
    st = dict(rows=rows, h=h, lc=lc, q_gate=rng.standard_normal((H_Q, 2 * D)).astype(np.float16),
              c_len=700)
    K, V, q = _brute_compressed(st, 700)
    want, lse = npref.attention(q, K, V, SCALE, N_REP)
    for splits in (1, 3):
        rc, out, _ = oracle_attn(st, num_splits=splits)
        got, glse = npref.triple_to_out(out)
        np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-5)
        np.testing.assert_allclose(glse, lse, atol=2e-5)


def test_attn_oracle_outliers_past_cap_and_mult_range():
    # ordinals >= 50 (sign -1, residual 0) and out-of-range multipliers (1):
    # the oracle's decode against the independent float64 decoder
    lc, h = layer_consts()
    rows = stressed_rows_np(120 * H_KV, seed=77)
    n_out = (((rows["kmask"][:, :, None] >> (2 * np.arange(16, dtype=np.uint32))) & 3) == 3).sum((1, 2))
    assert (n_out > 50).any() and (n_out == 256).any()
    rng = np.random.default_rng(78)
    st = dict(rows=rows, h=h, lc=lc, q_gate=rng.standard_normal((H_Q, 2 * D)).astype(np.float16),
              c_len=120)
    K, V, q = _brute_compressed(st, 120)
    want, lse = npref.attention(q, K, V, SCALE, N_REP)
    rc, out, _ = oracle_attn(st)
    assert rc == 0
    got, glse = npref.triple_to_out(out)
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-5)
    np.testing.assert_allclose(glse, lse, atol=2e-5)


def test_attn_oracle_start_pos_and_lq():
    st = two_region_state(seed=12)
    rc, out, _ = oracle_attn(st, c_len=200, start_pos=37)
    K, V, q = _brute_compressed(st, 200, start_pos=37)
    want, _ = npref.attention(q, K, V, SCALE, N_REP)
    np.testing.assert_allclose(npref.triple_to_out(out)[0], want, rtol=1e-4, atol=1e-5)
    # L_q = 3: query l sees tokens [0, l+1) and reads the same q row (ref .cu:1508-1512, 1542)
    rc, out3, _ = oracle_attn(st, c_len=200, L_q=3)
    assert rc == 0
    for l in range(3):
        K, V, q = _brute_compressed(st, l + 1)
        want, _ = npref.attention(q, K, V, SCALE, N_REP)
        got = npref.triple_to_out(out3.reshape(H_Q, 3, 258)[:, l])[0]
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_attn_zero_codes_uniform_softmax():
    lc, h = layer_consts()
    rows = random_rows_np(50 * H_KV, seed=8)
    rows["kmask"][:] = 0
    st = dict(rows=rows, h=h, lc=lc, q_gate=np.random.default_rng(9).standard_normal(
        (H_Q, 2 * D)).astype(np.float16), c_len=50)
    rc, out, _ = oracle_attn(st)
    np.testing.assert_allclose(out[:, 256], 0.0, atol=0)     # every score is 0
    np.testing.assert_allclose(out[:, 257], 50.0, rtol=1e-6)  # sum_exp = c_len
    _, V, _ = _brute_compressed(st, 50)
    want = np.stack([V[:, h // N_REP].mean(0) for h in range(H_Q)])
    np.testing.assert_allclose(npref.triple_to_out(out)[0], want, rtol=1e-4, atol=1e-5)


def test_attn_error_codes():
    st = two_region_state(seed=13)
    assert oracle_attn(st, c_len=0)[0] == -100
    r, h, lc = st["rows"], st["h"], st["lc"]
    rc, _, _ = oracle.attn(st["q_gate"], r["kpay"], r["vpay"], r["vsm"], r["kmask"], r["knorm"],
                           r["krn"], r["vnorm"], r["vrn"], h["cents_k"], h["cents_v"], h["vq"],
                           h["rotor_k"], h["rotor_v"], h["d_k"], h["d_v"], num_queries=H_Q,
                           num_heads=H_Q, L_q=1, c_len=10, n_rep=N_REP, scale=SCALE,
                           alpha_k=1.0, alpha_v=1.0, rope_base=THETA, start_pos=0,
                           num_splits=4, with_partial=False)
    assert rc == -101


def test_split_partition_lse_invariance():
    st = two_region_state(seed=14)
    outs = [npref.triple_to_out(oracle_attn(st, num_splits=s)[1])[0] for s in (1, 2, 7, 32, 48)]
    for o in outs[1:]:
        np.testing.assert_allclose(o, outs[0], rtol=1e-5, atol=1e-6)
    # empty splits (more splits than tokens): max -1e20, sum 0 in the partials
    rc, out, part = oracle_attn(st, c_len=5, num_splits=8)
    assert np.all(part[:, 5:, 256] == np.float32(-1e20)) and np.all(part[:, 5:, 257] == 0)


def test_window_and_merge_vs_union_softmax():
    st = two_region_state(seed=15)
    rc, wout = oracle_window(st)
    assert rc == 0
    Kw = npref.f16(st["k_roped"][st["c_len"]:])
    Vw = npref.f16(st["v"][st["c_len"]:])
    q = npref.f16(st["q_gate"])[:, :D]
    want_w, _ = npref.attention(q, Kw, Vw, SCALE, N_REP)
    np.testing.assert_allclose(npref.triple_to_out(wout)[0], want_w, rtol=1e-5, atol=1e-6)
    rc, cout, _ = oracle_attn(st)
    rc, merged = oracle.merge_gate(cout, wout, st["q_gate"], H_q=H_Q, has_w=True)
    Kc, Vc, _ = _brute_compressed(st, st["c_len"])
    want, _ = npref.attention(q, np.concatenate([Kc, Kw]), np.concatenate([Vc, Vw]), SCALE, N_REP)
    gate = npref.sigmoid(npref.f16(st["q_gate"])[:, D:])
    np.testing.assert_allclose(merged.astype(np.float64), want * gate, rtol=2e-3, atol=2e-3)
    # has_w = 0 uses the compressed triple alone
    rc, only_c = oracle.merge_gate(cout, None, st["q_gate"], H_q=H_Q, has_w=False)
    want_c, _ = npref.attention(q, Kc, Vc, SCALE, N_REP)
    np.testing.assert_allclose(only_c.astype(np.float64), want_c * gate, rtol=2e-3, atol=2e-3)


def test_window_wraps_ring():
    st = two_region_state(seed=16, n_tokens=600, boundary=384)  # window 216 slots, wraps
    st["win_start"], st["win_len"] = 384 % 256, 216
    rc, wout = oracle_window(st)
    Kw = npref.f16(st["k_roped"][384:600])
    Vw = npref.f16(st["v"][384:600])
    want, _ = npref.attention(npref.f16(st["q_gate"])[:, :D], Kw, Vw, SCALE, N_REP)
    np.testing.assert_allclose(npref.triple_to_out(wout)[0], want, rtol=1e-5, atol=1e-6)
    assert oracle.window_attn(st["q_gate"], st["ring_k"], st["ring_v"], win_start=0, win_len=0,
                              ring_cap=256, H_q=H_Q, H_kv=H_KV, scale=SCALE)[0] == -100


def test_gather_q():
    q = np.random.default_rng(0).standard_normal((H_Q, 2 * D)).astype(np.float16)
    rc, out = oracle.gather_q(q, H_q=H_Q)
    assert rc == 0 and np.array_equal(out, q[:, :D])


# ------------------------------------------- config-1 baseline (reference tests)
def _modular_inputs(H_q, H_kv, hd, max_seq):
    """The deterministic inputs of ref tests/test_gqa_attention_gpu.mojo:105-109."""
    i = np.arange(H_q * 2 * hd)
    qg = ((i * 7919 + 1013) % 2000).astype(np.float32) * 0.001 - 1.0
    j = np.arange(max_seq * H_kv * hd)
    k = ((j * 6271 + 5003) % 2000).astype(np.float32) * 0.001 - 1.0
    v = ((j * 4931 + 7919) % 2000).astype(np.float32) * 0.002 - 2.0
    return qg, k, v


def gqa_fp64(qg, k, v, seq, H_q, H_kv, hd, scale):
    """FP64 reference of ref tests/test_gqa_attention_gpu.mojo:36-84 (1/(Z+1e-9))."""
    grp = H_q // H_kv
    kd = H_kv * hd
    out = np.zeros(H_q * hd)
    for hq in range(H_q):
        hkv = hq // grp
        s = np.array([qg[hq * 2 * hd:hq * 2 * hd + hd] @ k[t * kd + hkv * hd:t * kd + hkv * hd + hd]
                      for t in range(seq)]) * scale
        e = np.exp(s - s.max())
        p = e / (e.sum() + 1e-9)
        ctx = p @ np.stack([v[t * kd + hkv * hd:t * kd + hkv * hd + hd] for t in range(seq)])
        out[hq * hd:(hq + 1) * hd] = ctx * npref.sigmoid(qg[hq * 2 * hd + hd:hq * 2 * hd + 2 * hd])
    return out


@pytest.mark.parametrize("H_q,H_kv,seq,max_seq", [(24, 4, 8, 16), (4, 2, 16, 16), (4, 2, 1, 16)])
def test_gqa_host_reference_cases(H_q, H_kv, seq, max_seq):
    qg, k, v = _modular_inputs(H_q, H_kv, 256, max_seq)
    qg16, k16, v16 = (a.astype(np.float16) for a in (qg, k, v))
    want = gqa_fp64(qg16.astype(np.float64), k16.astype(np.float64), v16.astype(np.float64),
                    seq, H_q, H_kv, 256, 1.0 / 16.0)
    got = oracle.gqa_host(qg16.reshape(H_q, 512), k16.reshape(max_seq, H_kv, 256),
                          v16.reshape(max_seq, H_kv, 256), seq_len=seq, H_q=H_q, H_kv=H_kv,
                          scale=1.0 / 16.0)
    rel = np.abs(got.ravel() - want).max() / np.abs(want).max()
    assert rel <= 2e-3  # the reference test's tolerance


@pytest.mark.parametrize("pos", [0, 1, 511, 8191])
def test_partial_rope_reference_cases(pos):
    """ref tests/test_rope_gpu.mojo:17-45: Bonsai dims (rot 64, theta 1e7, Q stride 512)."""
    H = 24
    j = np.arange(H * 512)
    x = (((j * 7919 + 1013) % 2000).astype(np.float32) * 0.002 - 2.0).astype(np.float16)
    got = oracle.partial_rope_fp16(x.reshape(H, 512), num_heads=H, head_dim=256, rotary_dim=64,
                                   pos=pos, theta=1e7, stride=512)
    xr = x.reshape(H, 512).astype(np.float64)
    want = xr.copy()
    want[:, :256] = npref.rope(xr[None, :, :256], [pos])[0]
    np.testing.assert_allclose(got.astype(np.float64), want, atol=2e-3, rtol=2e-3)
    assert np.array_equal(got[:, 64:], x.reshape(H, 512)[:, 64:])  # tail + gate untouched
    if pos == 0:
        assert np.array_equal(got, x.reshape(H, 512))


def test_rope_helper_matches_oracle_rope():
    """The test-side K RoPE equals the reference's partial_rope on fp16 rows."""
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, H_KV, D)).astype(np.float16)
    for pos in (0, 100, 4000):
        a = rope_fp16_rows(k, [pos])[0]
        b = oracle.partial_rope_fp16(k[0], num_heads=H_KV, head_dim=256, rotary_dim=64, pos=pos,
                                     theta=1e7)
        assert np.abs(a.astype(np.float32) - b.astype(np.float32)).max() <= 2e-3
