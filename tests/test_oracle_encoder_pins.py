"""Closed-form float64 pins of every scalar field the compressor writes.

The compressor (ref:src/csrc/qmv_sm75_kernel.cu:1256-1467) is restated line
by line in oracle/khq_oracle.c and the GPU kernel is tested bit-exact against
that restatement, so a mistake in the restatement would pass every GPU test.
These tests recompute each output field from an independent float64
projection (H_256 as an explicit matrix, 4x4 rotor products, numpy sums) and
require exact equality wherever the float64 value is not within float32
round-off of a rounding or comparison boundary:

K (.cu:1318-1351, 1429-1466): norm, c_base_mult = sum|p| / sum cb over codes
1 and 2 (dims past the 50-outlier cap count in neither sum), its clamp and
(u32)(mult * 1000) truncation, residual_j = max(0, |p_j ts| - cb_j mult),
rs = max(max_res, 1e-4) / 15, nibble_j = clamp(round(res_j / rs), 0, 15).
V (.cu:1353-1428): dim-3 code = argmin |p3 - a c_i| (first wins),
shared meta = max |p3 - a c|, dump = clamp(round(res / max(sm, 1e-4) * 7 + 8),
0, 15), vrn = sqrt(sum |p_012|^2 / (sum |a cb_code|^2 + 1e-8)).

Inputs are chosen so that a plausible slip fails: per-dim K centroids that
differ from dim to dim (a wrong cb index changes mult and residuals), ts != 1
(a dropped threshold scale changes residuals), and enough nibbles and dumps
with a fractional part above one half that truncation in place of roundf
fails.  Nothing here shares code with the oracle.
"""
import numpy as np

import npref
import oracle
from khqdata import D, layer_consts

F_S = 1.0 / 16.0
MARGIN = 2e-3  # float32 round-off of the oracle's sums, in units of the rounded quantity


def _proj64(x, d, rotor, alpha_unused=None):
    """p = (R_p^T . (H (x d / |x|)))_p / 16 in float64 (rot * f_s of .cu:1280-1305)."""
    x = np.asarray(x, np.float64)
    r = x * npref.f16(d)[None, :] / np.linalg.norm(x, axis=1, keepdims=True)
    r = r @ npref.H256.T
    R = npref.f16(rotor).reshape(64, 4, 4)  # rotor[p*16 + k*4 + c]
    return np.einsum("pkc,npk->npc", R, r.reshape(-1, 64, 4)).reshape(-1, D) * F_S


def _codes(kmask):
    dims = np.arange(D)
    return (kmask[:, dims // 16] >> (2 * (dims % 16)).astype(np.uint32)) & 3


def _round_half_up(v):
    return np.floor(v + 0.5)


def _near_half(v, m=MARGIN):
    f = v - np.floor(v)
    return np.abs(f - 0.5) < m


def _k_inputs(seed, n):
    lc, h = layer_consts()
    rng = np.random.default_rng(seed)
    cents = npref.f16(h["cents_k"]).reshape(4, D).copy()
    cents[2] = cents[2] * rng.uniform(0.6, 1.6, D)  # per-dim base centroids
    h = dict(h)
    h["cents_k"] = cents.astype(np.float16).reshape(-1)
    x = rng.standard_normal((n, D))
    # a third of the rows built from a projection with 30..90 large dims
    # (x = d * H (R p), the compress transform inverted), so some rows pass
    # the 50-outlier cap
    k = n // 3
    tgt = rng.standard_normal((k, D)) * 0.5
    for i in range(k):
        idx = rng.choice(D, 30 + (60 * i) // k, replace=False)
        tgt[i, idx] = rng.choice([-1.0, 1.0], len(idx)) * rng.uniform(2.0, 3.5, len(idx))
    R = npref.f16(h["rotor_k"]).reshape(64, 4, 4)
    r = np.einsum("pkc,npc->npk", R, tgt.reshape(k, 64, 4)).reshape(k, D)
    x[:k] = (r @ npref.H256.T) * npref.f16(h["d_k"])[None, :]
    return h, x.astype(np.float16)


def _k_expect(x, h, ts):
    """Float64 K fields: codes, mult, residual ratio res/rs, rs, plus margins."""
    p = _proj64(x, h["d_k"], h["rotor_k"])
    a = np.abs(p)
    cb = npref.f16(h["cents_k"]).reshape(4, D)[2]
    cand = a > 1.6 * F_S
    ordn = np.cumsum(cand, 1) - cand
    is3 = cand & (ordn < 50)
    normal = ~cand & (a > 0.47 * F_S)
    s_norm = (a * normal).sum(1)
    s_cb = (cb[None, :] * normal).sum(1)
    mult = np.where(s_cb > 1e-5, s_norm / np.where(s_cb > 0, s_cb, 1.0), 1.0)
    mult = np.where((mult < 0.1) | (mult > 10.0), 1.0, mult)
    res = np.where(is3, np.maximum(0.0, a * ts - cb[None, :] * mult[:, None]), 0.0)
    n_out = is3.sum(1)
    max_res = res.max(1)
    rs = np.where(n_out > 0, np.maximum(max_res, 1e-4) / 15.0, 0.0)
    return dict(p=p, is3=is3, mult=mult, res=res, rs=rs, n_out=n_out, cand=cand)


def test_k_scalar_fields_closed_form():
    h, x = _k_inputs(seed=21, n=96)
    ts = 1.3
    rc, kmask, knorm, krn, kpay, sm = oracle.compress(x, h["d_k"], h["rotor_k"], h["cents_k"],
                                                      h["cents_k"], ts=ts, alpha=1.0, is_v=False)
    assert rc == 0
    e = _k_expect(x, h, ts)
    codes = _codes(kmask)
    # rows whose code decisions are clear (thresholds 1.6 f_s and 0.47 f_s)
    a = np.abs(e["p"])
    clear = ((np.abs(a - 1.6 * F_S) > 1e-5) & (np.abs(a - 0.47 * F_S) > 1e-5)).all(1)
    assert clear.sum() > 80
    np.testing.assert_array_equal(codes[clear] == 3, e["is3"][clear])
    assert (e["cand"].sum(1) > 50).any(), "no row exercises the 50-outlier cap"

    # norm: fp16(sqrt(sum x^2 + 1e-8))
    xn = np.sqrt((x.astype(np.float64) ** 2).sum(1) + 1e-8)
    ok = np.float16(xn * (1 + 1e-6)) == np.float16(xn * (1 - 1e-6))
    np.testing.assert_array_equal(knorm[ok], xn[ok].astype(np.float16))

    # c_base_mult word: (u32)(mult * 1000), truncation of the float product
    word = kpay[:, 0:4].copy().view(np.uint32)[:, 0].astype(np.int64)
    m1000 = e["mult"] * 1000.0
    f = m1000 - np.floor(m1000)
    okm = clear & (f > MARGIN * 5) & (f < 1 - MARGIN * 5)
    assert okm.sum() > 60
    np.testing.assert_array_equal(word[okm], np.floor(m1000[okm]).astype(np.int64))
    assert (e["mult"][clear] != 1.0).all()  # the computed ratio, not the default

    # residual scale: fp16(max(max_res, 1e-4) / 15), 0 without outliers
    rs = e["rs"]
    okr = clear & (np.float16(rs * (1 + 1e-5)) == np.float16(rs * (1 - 1e-5)))
    assert okr.sum() > 60
    np.testing.assert_array_equal(krn[okr], rs[okr].astype(np.float16))

    # nibbles of outlier ordinals j < n_out: clamp(round(res / rs), 0, 15);
    # past n_out the 25 nibble bytes stay zero
    nib = np.stack([(kpay[:, 4 + j // 2] >> (4 * (j % 2))) & 0xF for j in range(50)], 1)
    n_cmp = n_trunc_differs = 0
    for i in np.nonzero(clear)[0]:
        k = e["n_out"][i]
        assert np.all(nib[i, k:] == 0)
        if k == 0:
            continue
        ratio = e["res"][i][e["is3"][i]] / rs[i]  # ordinal order = dim order
        want = np.clip(_round_half_up(ratio), 0, 15)
        safe = ~_near_half(ratio)
        np.testing.assert_array_equal(nib[i, :k][safe], want[safe].astype(np.uint8))
        n_cmp += safe.sum()
        n_trunc_differs += (safe & (np.floor(ratio) != want)).sum()
        # the largest residual takes nibble 15 (rs = max_res / 15)
        if e["res"][i].max() > 1e-4:
            assert nib[i, :k].max() == 15
    assert n_cmp > 500 and n_trunc_differs > 100, (n_cmp, n_trunc_differs)

    # sign bits: 1 where p > 0, for ordinals < n_out; marker byte and tail
    for i in np.nonzero(clear)[0][:32]:
        dims = np.nonzero(e["is3"][i])[0]
        bits = [(kpay[i, 29 + j // 8] >> (j % 8)) & 1 for j in range(len(dims))]
        assert bits == [int(e["p"][i, d] > 0) for d in dims]
        tail = [(kpay[i, 29 + j // 8] >> (j % 8)) & 1 for j in range(len(dims), 56)]
        assert not any(tail)
    assert np.all(kpay[:, 36] == 2) and np.all(kpay[:, 37:] == 0)
    assert np.all(sm.view(np.uint32) == 0)


def test_k_mult_defaults_and_clamp():
    # rows whose normal dims' mean |p| / cb is outside [0.1, 10] take mult 1.0:
    # scale the base centroids instead of the data
    lc, h = layer_consts()
    rng = np.random.default_rng(22)
    x = rng.standard_normal((8, D)).astype(np.float16)
    for scale, clamped in ((1.0, False), (1e-3, True), (30.0, True)):
        cents = npref.f16(h["cents_k"]).reshape(4, D).copy()
        cents[2] *= scale
        hh = dict(h, cents_k=cents.astype(np.float16).reshape(-1))
        rc, _, _, _, kpay, _ = oracle.compress(x, hh["d_k"], hh["rotor_k"], hh["cents_k"],
                                               hh["cents_k"], ts=1.0, alpha=1.0, is_v=False)
        word = kpay[:, 0:4].copy().view(np.uint32)[:, 0]
        e = _k_expect(x, hh, 1.0)
        if clamped:
            assert np.all(word == 1000)
        else:
            assert np.all(word != 1000)
            np.testing.assert_allclose(word, np.floor(e["mult"] * 1000), atol=1)


def test_v_scalar_fields_closed_form():
    alpha = 1.0 / 16.0
    lc, h = layer_consts(alpha_v=alpha)
    rng = np.random.default_rng(23)
    x = rng.standard_normal((64, D)).astype(np.float16)
    rc, _, vnorm, vrn, vpay, vsm = oracle.compress(x, h["d_v"], h["rotor_v"], h["cents_v"],
                                                   h["vq"], ts=1.95, alpha=alpha, is_v=True)
    assert rc == 0
    p = _proj64(x, h["d_v"], h["rotor_v"]).reshape(-1, 64, 4)
    code, d3c, dump = npref.unpack_v_fields(vpay)
    cv = npref.f16(h["cents_v"]).reshape(4, D)[:2, np.arange(64) * 4 + 3] * alpha  # [2, 64]

    # norm
    xn = np.sqrt((x.astype(np.float64) ** 2).sum(1) + 1e-8)
    ok = np.float16(xn * (1 + 1e-6)) == np.float16(xn * (1 - 1e-6))
    np.testing.assert_array_equal(vnorm[ok], xn[ok].astype(np.float16))

    # dim-3 code: argmin |p3 - a c_i| over i = 0, 1, the first on ties
    d0 = np.abs(p[:, :, 3] - cv[0][None, :])
    d1 = np.abs(p[:, :, 3] - cv[1][None, :])
    want_c = np.where(d1 < d0, 1, 0)
    clear = np.abs(d1 - d0) > 1e-6
    np.testing.assert_array_equal(d3c[clear], want_c[clear])

    # shared meta: max |residual| (float32), residual = p3 - a c_code
    res = p[:, :, 3] - cv[d3c, np.arange(64)[None, :]]
    max_res = np.abs(res).max(1)
    smv = vsm.copy().view(np.float32).ravel().astype(np.float64)
    np.testing.assert_allclose(smv, max_res, rtol=2e-6)

    # dump: clamp(round(res / max(sm, 1e-4) * 7 + 8), 0, 15)
    scaled = res / np.maximum(max_res, 1e-4)[:, None] * 7.0 + 8.0
    want_d = np.clip(_round_half_up(scaled), 0, 15)
    safe = ~_near_half(scaled)
    assert safe.mean() > 0.95
    np.testing.assert_array_equal(dump[safe], want_d[safe])
    assert (safe & (np.floor(scaled) != want_d)).sum() > 500  # truncation would fail
    # the largest |residual| of each row sits at dump 1 or 15
    amax = np.abs(res).argmax(1)
    ext = dump[np.arange(64), amax]
    assert np.all((ext == 15) | (ext == 1))

    # energy correction: sqrt(sum |p_012|^2 / (sum |a cb_code|^2 + 1e-8)), fp16
    cb = npref.f16(h["vq"]).reshape(64, 256, 3)
    sel = cb[np.arange(64)[None, :], code] * alpha  # [n, 64, 3]
    e_true = (p[:, :, :3] ** 2).sum((1, 2))
    e_vq = (sel ** 2).sum((1, 2))
    want_rn = np.sqrt(e_true / (e_vq + 1e-8))
    okr = np.float16(want_rn * (1 + 1e-5)) == np.float16(want_rn * (1 - 1e-5))
    assert okr.sum() > 50
    np.testing.assert_array_equal(vrn[okr], want_rn[okr].astype(np.float16))
    # an inverted ratio would not match: the data keep it away from 1
    assert np.abs(np.log(want_rn)).min() > 1e-2


def test_v_dump_scale_floor():
    # rows whose dim-3 projections sit within ~1e-4 of a centroid: max_res is
    # below the 1e-4 floor of the dump scale, so dump = round(res / 1e-4 * 7 + 8)
    alpha = 1.0 / 16.0
    lc, h = layer_consts(alpha_v=alpha)
    rng = np.random.default_rng(24)
    n = 16
    cv = npref.f16(h["cents_v"]).reshape(4, D)[:2, np.arange(64) * 4 + 3] * alpha
    t = np.zeros((n, 64, 4))
    t[:, :, 3] = cv[rng.integers(0, 2, (n, 64)), np.arange(64)[None, :]]
    t[:, :, 3] += rng.uniform(-4e-5, 4e-5, (n, 64))
    rest = rng.standard_normal((n, 64, 3))
    room = 1.0 - (t[:, :, 3] ** 2).sum(1)
    t[:, :, :3] = rest * np.sqrt(room / (rest ** 2).sum((1, 2)))[:, None, None]
    assert np.allclose((t ** 2).sum((1, 2)), 1.0)
    R = npref.f16(h["rotor_v"]).reshape(64, 4, 4)
    r = np.einsum("pkc,npc->npk", R, t).reshape(n, D)
    x = ((r @ npref.H256.T) * npref.f16(h["d_v"])[None, :]).astype(np.float16)
    rc, _, _, _, vpay, vsm = oracle.compress(x, h["d_v"], h["rotor_v"], h["cents_v"], h["vq"],
                                             ts=1.95, alpha=alpha, is_v=True)
    p = _proj64(x, h["d_v"], h["rotor_v"]).reshape(-1, 64, 4)
    _, d3c, dump = npref.unpack_v_fields(vpay)
    res = p[:, :, 3] - cv[d3c, np.arange(64)[None, :]]
    max_res = np.abs(res).max(1)
    assert max_res.max() < 1e-4
    np.testing.assert_allclose(vsm.copy().view(np.float32).ravel(), max_res, rtol=1e-3)
    scaled = res / 1e-4 * 7.0 + 8.0
    want = np.clip(_round_half_up(scaled), 0, 15)
    safe = ~_near_half(scaled, 0.05)
    np.testing.assert_array_equal(dump[safe], want[safe])
    assert (want[safe] != 8).sum() > 100
