"""Seeded host-side (numpy) test states shared by the CPU and GPU tests."""
from __future__ import annotations

import numpy as np

import oracle
from khq import centroids as C

D = 256
H_Q, H_KV, N_REP = 24, 4, 6
SCALE = 1.0 / 16.0
THETA = 1e7


def layer_consts(layer_id=3, seed=1234, **kw):
    lc = C.synthetic_layer(layer_id, seed=seed, **kw)
    return lc, lc.fp16()


def rope_fp16_rows(x, positions, theta=THETA):
    """RoPE (fp32 math, fp16 out) of x [T, H, 256] at positions, the way the
    caller ropes K before the ring write (partial_rope, half-split)."""
    half = 32
    m = np.arange(half, dtype=np.float32)
    freq = np.exp(np.float32(np.log(theta)) * (-2.0 * m / 64.0)).astype(np.float32)
    ang = (np.asarray(positions, np.float32)[:, None] * freq[None, :]).astype(np.float32)
    c = np.cos(ang)[:, None, :].astype(np.float32)
    s = np.sin(ang)[:, None, :].astype(np.float32)
    xf = x.astype(np.float32)
    out = xf.copy()
    out[..., :half] = xf[..., :half] * c - xf[..., half:64] * s
    out[..., half:64] = xf[..., :half] * s + xf[..., half:64] * c
    return out.astype(np.float16)


def compress_rows(x_tokens, h, is_v):
    """Oracle-compress tokens [T, H_kv, 256] -> packed rows (row = t*H_kv + hkv)."""
    T, hkv, _ = x_tokens.shape
    x = np.ascontiguousarray(x_tokens.reshape(T * hkv, D))
    if is_v:
        rc, mask, nrm, rn, pay, sm = oracle.compress(x, h["d_v"], h["rotor_v"], h["cents_v"],
                                                     h["vq"], ts=1.95, alpha=1.0, is_v=True)
    else:
        rc, mask, nrm, rn, pay, sm = oracle.compress(x, h["d_k"], h["rotor_k"], h["cents_k"],
                                                     h["cents_k"], ts=1.0, alpha=1.0, is_v=False)
    assert rc == 0
    return mask, nrm, rn, pay, sm


def two_region_state(seed=7, n_tokens=512, boundary=384, lc_kw=None):
    """State after n_tokens decode steps with the reference cadence: rows for
    tokens [0, boundary), ring holding tokens [n_tokens-256, n_tokens)."""
    lc, h = layer_consts(**(lc_kw or {}))
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_tokens, H_KV, D)).astype(np.float16)
    v = rng.standard_normal((n_tokens, H_KV, D)).astype(np.float16)
    k_roped = rope_fp16_rows(k, np.arange(n_tokens))
    kmask, knorm, krn, kpay, _ = compress_rows(k[:boundary], h, False)
    _, vnorm, vrn, vpay, vsm = compress_rows(v[:boundary], h, True)
    ring_k = np.zeros((256, H_KV, D), np.float16)
    ring_v = np.zeros((256, H_KV, D), np.float16)
    ring_u = np.zeros((256, H_KV, D), np.float16)
    for t in range(max(0, n_tokens - 256), n_tokens):
        ring_k[t % 256] = k_roped[t]
        ring_v[t % 256] = v[t]
        ring_u[t % 256] = k[t]
    q_gate = rng.standard_normal((H_Q, 2 * D)).astype(np.float16)
    rows = dict(kmask=kmask, kpay=kpay, knorm=knorm, krn=krn, vpay=vpay, vnorm=vnorm, vrn=vrn,
                vsm=vsm)
    return dict(lc=lc, h=h, rows=rows, ring_k=ring_k, ring_v=ring_v, ring_u=ring_u,
                q_gate=q_gate, k=k, v=v, k_roped=k_roped, c_len=boundary,
                win_start=boundary % 256, win_len=n_tokens - boundary)


def oracle_attn(st, c_len=None, num_splits=1, rope_base=THETA, L_q=1, start_pos=0):
    r, h, lc = st["rows"], st["h"], st["lc"]
    c_len = st["c_len"] if c_len is None else c_len
    return oracle.attn(st["q_gate"], r["kpay"], r["vpay"], r["vsm"], r["kmask"], r["knorm"],
                       r["krn"], r["vnorm"], r["vrn"], h["cents_k"], h["cents_v"], h["vq"],
                       h["rotor_k"], h["rotor_v"], h["d_k"], h["d_v"],
                       num_queries=H_Q * L_q, num_heads=H_Q, L_q=L_q, c_len=c_len,
                       n_rep=N_REP, scale=SCALE, alpha_k=lc.alpha_k, alpha_v=lc.alpha_v,
                       rope_base=rope_base, start_pos=start_pos, num_splits=num_splits)


def oracle_window(st):
    return oracle.window_attn(st["q_gate"], st["ring_k"], st["ring_v"],
                              win_start=st["win_start"], win_len=st["win_len"], ring_cap=256,
                              H_q=H_Q, H_kv=H_KV, scale=SCALE)


def random_rows_np(rows, seed):
    """numpy twin of khq.synth.random_rows (same spec, own generator)."""
    rng = np.random.default_rng(seed)
    n_out = rng.integers(0, 51, (rows, 1))
    rank = rng.random((rows, D)).argsort(1).argsort(1)
    codes = rng.integers(0, 3, (rows, D))
    codes = np.where(rank < n_out, 3, codes).astype(np.uint64)
    words = (codes.reshape(rows, 16, 16) << (2 * np.arange(16, dtype=np.uint64))).sum(2)
    kmask = words.astype(np.uint32)
    kpay = rng.integers(0, 256, (rows, 40)).astype(np.uint8)
    mult = rng.integers(100, 10001, rows).astype(np.uint32)
    kpay[:, 0:4] = mult.view(np.uint8).reshape(rows, 4)
    kpay[:, 36] = 2
    kpay[:, 37:40] = 0
    vpay = rng.integers(0, 256, (rows, 104)).astype(np.uint8)
    return dict(kmask=kmask, kpay=kpay,
                knorm=rng.uniform(0.5, 2.0, rows).astype(np.float16),
                krn=rng.uniform(0.002, 0.008, rows).astype(np.float16),
                vpay=vpay, vnorm=rng.uniform(0.5, 2.0, rows).astype(np.float16),
                vrn=rng.uniform(0.8, 1.2, rows).astype(np.float16),
                vsm=rng.uniform(0.01, 0.05, rows).astype(np.float32).view(np.uint8).reshape(rows, 4))


def stressed_rows_np(rows, seed):
    """random_rows_np with rows the compressor never writes but the format
    defines: more than 50 code-3 dims (ordinals >= 50 decode with sign -1 and
    residual 0; up to every dim an outlier) and stored multipliers outside
    [0.1, 10] (read as 1)."""
    r = random_rows_np(rows, seed)
    rng = np.random.default_rng(seed + 1)
    n_out = rng.choice([0, 49, 50, 51, 64, 128, 200, 256], size=rows)
    rank = rng.random((rows, D)).argsort(1).argsort(1)
    codes = rng.integers(0, 3, (rows, D))
    codes = np.where(rank < n_out[:, None], 3, codes).astype(np.uint64)
    words = (codes.reshape(rows, 16, 16) << (2 * np.arange(16, dtype=np.uint64))).sum(2)
    r["kmask"] = words.astype(np.uint32)
    mraw = rng.choice(np.array([0, 99, 100, 5000, 10000, 10001, 0xFFFFFFFF], dtype=np.uint32),
                      size=rows)
    r["kpay"][:, 0:4] = mraw.view(np.uint8).reshape(rows, 4)
    return r

