"""Independent float64 numpy reading of the KHQ formats and attention.

Used only to pin the C oracle: it decodes the packed rows straight from the
format description (ref:src/csrc/qmv_sm75_kernel.cu:1409-1465 for packing,
the independent unpacker of :2962-3024 for the V 12-bit fields), builds the
full K/V rows with an explicit Hadamard matrix and per-patch 4x4 products,
applies RoPE, and runs textbook softmax attention in float64.  Nothing here
shares code with the oracle or the kernels.
"""
from __future__ import annotations

import numpy as np
from scipy.linalg import hadamard

D = 256
NP = 64
H256 = hadamard(D).astype(np.float64)


def f16(a):
    return np.asarray(a, np.float16).astype(np.float64)


def decode_k(kmask, kpay, knorm, krn, cents_k, rotor_k, d_k, alpha_k):
    """Pre-RoPE K rows [n, 256] (float64) from packed K rows."""
    kmask = np.asarray(kmask).view(np.uint32).reshape(-1, 16)
    n = kmask.shape[0]
    kpay = np.asarray(kpay, np.uint8).reshape(n, 40)
    dims = np.arange(D)
    codes = (kmask[:, dims // 16] >> (2 * (dims % 16)).astype(np.uint32)) & 3  # [n,256]
    is3 = codes == 3
    ordinal = np.cumsum(is3, axis=1) - is3  # number of code-3 dims before i
    mult = kpay[:, 0:4].copy().view(np.uint32)[:, 0].astype(np.float32) / np.float32(1000.0)
    mult = np.where((mult < 0.1) | (mult > 10.0) | np.isnan(mult), np.float32(1.0), mult)
    mult = mult.astype(np.float64)
    cb = f16(np.asarray(cents_k).reshape(4, D)[2])
    rs = f16(krn).reshape(n, 1)
    j = np.minimum(ordinal, 49)
    rows = np.arange(n)[:, None]
    nib = (kpay[rows, 4 + j // 2] >> ((j % 2) * 4).astype(np.uint8)) & 0xF
    sbit = (kpay[rows, 29 + j // 8] >> (j % 8).astype(np.uint8)) & 1
    valid = ordinal < 50
    sign = np.where(valid & (sbit == 1), 1.0, -1.0)
    res = np.where(valid, nib.astype(np.float64), 0.0)
    cbase = cb[None, :] * mult[:, None]
    val = np.where(codes == 2, cbase, 0.0)
    val = np.where(codes == 1, -cbase, val)
    val = np.where(is3, sign * (cbase + res * rs), val)
    val = val * alpha_k * f16(knorm).reshape(n, 1)
    R = f16(rotor_k).reshape(NP, 4, 4)  # R[p][c][k] = rotor[p*16 + c*4 + k]
    y = np.einsum("pck,npk->npc", R, val.reshape(n, NP, 4)).reshape(n, D)
    k = y @ H256.T
    return k / 256.0 / f16(d_k)[None, :]


def unpack_v_fields(vpay):
    """12-bit patch fields [n, 64] and VQ codes, unpacked group by group the
    way ref .cu:2976-2988 reads them."""
    w = np.asarray(vpay, np.uint8).reshape(-1, 104).copy().view(np.uint32).astype(np.uint64)
    n = w.shape[0]
    pv = np.zeros((n, NP), np.uint64)
    for g in range(8):
        w0, w1, w2 = w[:, g * 3], w[:, g * 3 + 1], w[:, g * 3 + 2]
        pv[:, g * 8 + 0] = w0 & 0xFFF
        pv[:, g * 8 + 1] = (w0 >> 12) & 0xFFF
        pv[:, g * 8 + 2] = (w0 >> 24) | ((w1 & 0xF) << 8)
        pv[:, g * 8 + 3] = (w1 >> 4) & 0xFFF
        pv[:, g * 8 + 4] = (w1 >> 16) & 0xFFF
        pv[:, g * 8 + 5] = (w1 >> 28) | ((w2 & 0xFF) << 4)
        pv[:, g * 8 + 6] = (w2 >> 8) & 0xFFF
        pv[:, g * 8 + 7] = (w2 >> 20) & 0xFFF
    p = np.arange(NP)
    hb = np.where(p < 32, (w[:, 24:25] >> (p % 32).astype(np.uint64)) & 1,
                  (w[:, 25:26] >> (p % 32).astype(np.uint64)) & 1)
    code = (pv & 0x7F) | (hb << 7)
    d3c = (pv >> 7) & 1
    dump = (pv >> 8) & 0xF
    return code.astype(np.int64), d3c.astype(np.int64), dump.astype(np.int64)


def decode_v(vpay, vnorm, vrn, vsm, cents_v, rotor_v, d_v, vq, alpha_v):
    """V rows [n, 256] (float64) from packed V rows."""
    code, d3c, dump = unpack_v_fields(vpay)
    n = code.shape[0]
    norm = f16(vnorm).reshape(n, 1)
    rn = f16(vrn).reshape(n, 1)
    sm = np.asarray(vsm, np.uint8).reshape(n, 4).copy().view(np.float32).astype(np.float64)
    cbk = f16(vq).reshape(NP, 256, 3)
    p = np.arange(NP)
    vrot = np.zeros((n, NP, 4))
    vrot[:, :, :3] = cbk[p[None, :], code] * alpha_v * norm[:, :, None] * rn[:, :, None]
    cv = f16(np.asarray(cents_v).reshape(4, D))[:, p * 4 + 3] * alpha_v  # [4, NP]
    vrot[:, :, 3] = cv[d3c, p[None, :]] * norm + (dump - 8.0) / 7.0 * sm * norm
    R = f16(rotor_v).reshape(NP, 4, 4)
    y = np.einsum("pck,npk->npc", R, vrot).reshape(n, D)
    return (y @ H256.T) / 16.0 / f16(d_v)[None, :]


def rope(k, positions, theta=1e7, rot=64, freq_mode="pow"):
    """Half-split RoPE (pairs i, i+32) on dims 0..rot-1 of k [..., T, H, D]
    at `positions` [T], float64."""
    half = rot // 2
    m = np.arange(half)
    freq = theta ** (-2.0 * m / rot)
    ang = np.asarray(positions, np.float64)[:, None] * freq[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    out = np.array(k, np.float64, copy=True)
    x0, x1 = out[..., :half].copy(), out[..., half:rot].copy()
    out[..., :half] = x0 * c - x1 * s
    out[..., half:rot] = x0 * s + x1 * c
    return out


def attention(q, K, V, scale, n_rep):
    """q [H_q, 256], K/V [T, H_kv, 256] -> (out [H_q,256], lse [H_q]) float64."""
    H_q = q.shape[0]
    out = np.zeros((H_q, D))
    lse = np.zeros(H_q)
    for h in range(H_q):
        kv = h // n_rep
        s = K[:, kv, :] @ q[h] * scale
        m = s.max()
        p = np.exp(s - m)
        l = p.sum()
        out[h] = (p @ V[:, kv, :]) / l
        lse[h] = m + np.log(l)
    return out, lse


def triple_to_out(tr):
    """Unnormalised (acc, max, sum_exp) [H, 258] -> (acc / sum_exp, lse)."""
    tr = np.asarray(tr, np.float64)
    return tr[:, :D] / tr[:, D + 1:D + 2], tr[:, D] + np.log(tr[:, D + 1])


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))
