"""CPU restatement of the KHQ calibration steps (test infrastructure only).

numpy versions of launch_cal_op ops 1-7 and 10, of the SmartK / SmartV
round trips and of the SmartVQ trainer (ref:src/csrc/qmv_sm75_kernel.cu:
2019-2085, 2089-2600, 2645-2681, 2722-3025, 3071-3349, 4434-4810), written
from the reference's algorithm in float64 so they can check the GPU steps
(tests/test_gpu_calib.py); each is itself pinned in tests/test_calib_ref.py
against closed forms (explicit Hadamard matrix, numpy eigh, SVD polar
factor, Lloyd fixed points, the independent format decoders of
tests/npref.py (the SmartV round trip also against a scalar restatement
of the reference's encoder loops), synthetic error landscapes with known
minima for the ops 8 / 9 search, central differences of the SmartVQ loss and of its
straight-through surrogate, Adam's closed-form first steps).  Nothing in the
product imports this file.
"""
from __future__ import annotations

import numpy as np
from scipy.linalg import hadamard

D, NP = 256, 64
FS = 0.0625
H256 = hadamard(D).astype(np.float64)


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float64)


def fwht_base(x, d):
    """op 1 (.cu:2019-2070): norms, FWHT(x fp16(d) / (norm + 1e-8)) / 16."""
    x = np.asarray(x, np.float64)
    n = np.sqrt((x * x).sum(1) + 1e-8)
    r = x * f16(d)[None, :] / (n[:, None] + 1e-8)
    return n, (r @ H256.T) * FS


def rotate(x, rp):
    """op 3 (.cu:2073-2085): out[p][c] = sum_k x[p][k] rp[16p + 4k + c]."""
    R = np.asarray(rp, np.float64).reshape(NP, 4, 4)
    return np.einsum("npk,pkc->npc", np.asarray(x, np.float64).reshape(-1, NP, 4), R).reshape(-1, D)


def k_static(proj):
    """op 2 (.cu:2645-2681)."""
    sg = np.asarray(proj, np.float64).std(0)
    c0 = 0.935 * sg
    ts = 16.0 / np.sqrt((0.528756 * c0 * c0 + 0.464545 * sg * sg).sum())
    c = 0.935 * sg * ts
    return np.stack([np.zeros(D), -c, c, c]), ts


def pca_rotors(base):
    """op 4 (.cu:3071-3145) by eigh: rotor column c = eigenvector of rank
    {1, 2, 3, 0}[c] by decreasing eigenvalue of the uncentred moment + 1e-3 I."""
    b = np.asarray(base, np.float64).reshape(-1, NP, 4)
    out = np.zeros((NP, 4, 4))
    for p in range(NP):
        m = b[:, p].T @ b[:, p] + 1e-3 * np.eye(4)
        w, v = np.linalg.eigh(m)
        order = np.argsort(-w)
        for c, s in enumerate((1, 2, 3, 0)):
            out[p, :, c] = v[:, order[s]]
    return out.reshape(NP, 16)


def kmeans4(data, iters=20):
    """op 5 (.cu:3147-3183): per dim, init (mn + (mx - mn) k / 3) * 0.8,
    Lloyd, first minimum wins, empty cluster -> 0."""
    x = np.asarray(data, np.float64)
    mn, mx = x.min(0), x.max(0)
    c = np.stack([(mn + (mx - mn) * (k / 3.0)) * 0.8 for k in range(4)])  # [4, D]
    for _ in range(iters):
        dist = (x[None, :, :] - c[:, None, :]) ** 2       # [4, rows, D]
        a = np.argmin(dist, 0)                             # first minimum
        new = np.zeros_like(c)
        for k in range(4):
            m = a == k
            cnt = m.sum(0)
            new[k] = np.where(cnt > 0, (x * m).sum(0) / np.maximum(cnt, 1), 0.0)
        c = new
    return c


def xorshift_rows(seed, rows):
    """op 6 initial codeword rows: per entry i = 256 p + k, s = seed ^ (i *
    2654435761 + 1) (u32), one xorshift, idx = (s & 0xFFFFFF) / 2^24 * rows."""
    i = np.arange(NP * 256, dtype=np.uint64)
    s = (np.uint64(seed) ^ ((i * np.uint64(2654435761) + np.uint64(1)) & np.uint64(0xFFFFFFFF)))
    s &= np.uint64(0xFFFFFFFF)
    s ^= (s << np.uint64(13)) & np.uint64(0xFFFFFFFF)
    s ^= s >> np.uint64(17)
    s ^= (s << np.uint64(5)) & np.uint64(0xFFFFFFFF)
    u = (s & np.uint64(0xFFFFFF)).astype(np.float32) / np.float32(16777216.0)
    idx = (u * np.float32(rows)).astype(np.int64)
    return np.minimum(idx, rows - 1).reshape(NP, 256)


def nearest(v3, cb):
    """first-minimum nearest codeword: v3 [n, 3], cb [256, 3]."""
    d = ((v3[:, None, :] - cb[None, :, :]) ** 2).sum(-1)
    return np.argmin(d, 1)


def kmeans_vq(rot, seed, iters=30):
    """op 6 (.cu:3185-3249)."""
    x = np.asarray(rot, np.float64).reshape(-1, NP, 4)
    idx = xorshift_rows(seed, x.shape[0])
    C = np.stack([x[idx[p], p, :3] for p in range(NP)])  # [NP, 256, 3]
    for _ in range(iters):
        for p in range(NP):
            a = nearest(x[:, p, :3], C[p])
            cnt = np.bincount(a, minlength=256)
            for c in range(3):
                s = np.bincount(a, weights=x[:, p, c], minlength=256)
                C[p, :, c] = np.where(cnt > 0, s / np.maximum(cnt, 1), C[p, :, c])
    return C


def polar_ns(M, iters=12):
    """Newton-Schulz polar iteration of ref .cu:3308-3349: X = M / |M|_F,
    X <- X (3 I - X^T X) / 2; kept as M's orthogonal polar factor's
    approximation (tests pin it against the SVD polar factor)."""
    X = np.asarray(M, np.float64) / np.sqrt((np.asarray(M, np.float64) ** 2).sum() + 1e-8)
    for _ in range(iters):
        X = 0.5 * X @ (3.0 * np.eye(4) - X.T @ X)
    return X


def procrustes(base, vq, rp, iters):
    """op 7 (.cu:3266-3349): target = nearest codeword (dims 0..2) of the
    rotated row plus its own dim 3, M = base^T target per patch, rotor =
    polar_ns(M)."""
    b = np.asarray(base, np.float64)
    R = np.asarray(rp, np.float64).reshape(NP, 16).copy()
    vq = np.asarray(vq, np.float64).reshape(NP, 256, 3)
    for _ in range(iters):
        rot = rotate(b, R).reshape(-1, NP, 4)
        tgt = rot.copy()
        for p in range(NP):
            tgt[:, p, :3] = vq[p][nearest(rot[:, p, :3], vq[p])]
        bb = b.reshape(-1, NP, 4)
        for p in range(NP):
            R[p] = polar_ns(bb[:, p].T @ tgt[:, p]).reshape(16)
    return R


def roundtrip_k(proj, norms, cents, rp, d, alpha):
    """SmartK round trip (.cu:2722-2862 as the tournament runs it): codes
    from |p| > 1.6 f_s (sign) or +-0.47 f_s, never code 3; mult over codes
    1, 2; decode sign * cents[2] * mult * alpha * norm -> R -> H -> / (256 d)."""
    p = np.asarray(proj, np.float64)
    cb = np.asarray(cents, np.float64).reshape(4, D)[2]
    a = np.abs(p)
    sg = np.where(a > 1.6 * FS, np.sign(p), np.where(p > 0.47 * FS, 1.0, np.where(p < -0.47 * FS, -1.0, 0.0)))
    nz = sg != 0
    sn = (a * nz).sum(1)
    sc = (f16(cb)[None, :] * nz).sum(1)
    mult = np.where(sc > 1e-5, sn / np.where(sc > 0, sc, 1), 1.0)
    mult = np.where((mult < 0.1) | (mult > 10), 1.0, mult)
    m2 = np.floor(mult.astype(np.float32) * np.float32(1000.0)).astype(np.float64) / 1000.0
    m2 = np.where((m2 < 0.1) | (m2 > 10), 1.0, m2)
    kv = sg * cb[None, :] * m2[:, None] * alpha * np.asarray(norms, np.float64)[:, None]
    R = np.asarray(rp, np.float64).reshape(NP, 4, 4)  # [p][k][c]
    y = np.einsum("pck,npk->npc", R, kv.reshape(-1, NP, 4)).reshape(-1, D)
    return (y @ H256.T) / (256.0 * np.asarray(d, np.float64)[None, :])


def dim_weights(x):
    x = np.asarray(x, np.float64)
    m = np.abs(x).mean(0)
    v = x.var(0)
    return m / (m.sum() + 1e-8), v / (v.sum() + 1e-8)


def roundtrip_v(proj, norms, cents, vq, rp, d, alpha):
    """SmartV round trip (.cu:2863-3025): per patch the nearest fp16(vq) *
    alpha codeword (first minimum), dim-3 code by |p3 - a c| (ties to 1),
    dump = clamp(round(res / max(g, 1e-4) * 7 + 8)), energy correction
    rounded to fp16; decode with the unrounded tables -> R -> H -> / (16 d)."""
    p = np.asarray(proj, np.float64).reshape(-1, NP, 4)
    n = p.shape[0]
    cbf = np.asarray(vq, np.float64).reshape(NP, 256, 3)
    cb16 = f16(cbf) * alpha
    cv = np.asarray(cents, np.float64).reshape(4, D)[:2, np.arange(NP) * 4 + 3]  # [2, NP]
    out = np.zeros((n, NP, 4))
    te = (p[:, :, :3] ** 2).sum((1, 2))
    code = np.stack([nearest(p[:, q, :3], cb16[q]) for q in range(NP)], 1)  # [n, NP]
    sel16 = cb16[np.arange(NP)[None, :], code]
    ve = (sel16 ** 2).sum((1, 2))
    rn = f16(np.sqrt(te / (ve + 1e-8)))
    c0, c1 = f16(cv[0]) * alpha, f16(cv[1]) * alpha
    d3 = np.where(np.abs(p[:, :, 3] - c0) < np.abs(p[:, :, 3] - c1), 0, 1)
    res = p[:, :, 3] - np.where(d3 == 0, c0, c1)
    g = np.abs(res).max(1)
    rsc = np.maximum(g, 1e-4)
    x = res / rsc[:, None] * 7.0 + 8.0
    dump = np.clip(np.where(x >= 0, np.floor(x + 0.5), -np.floor(-x + 0.5)), 0, 15)
    nr = np.asarray(norms, np.float64)
    out[:, :, :3] = cbf[np.arange(NP)[None, :], code] * alpha * (nr * rn)[:, None, None]
    cvd = np.where(d3 == 0, cv[0][None, :], cv[1][None, :]) * alpha
    out[:, :, 3] = cvd * nr[:, None] + (dump - 8.0) / 7.0 * (g * nr)[:, None]
    R = np.asarray(rp, np.float64).reshape(NP, 4, 4)
    y = np.einsum("pck,npk->npc", R, out).reshape(n, D)
    return (y @ H256.T) / (16.0 * np.asarray(d, np.float64)[None, :])


def tournament(x32, x16, d, rp, cents, ts0, vq=None):
    """ops 8 (vq None: K) and 9 (V) in float64: returns (ts, alpha)."""
    wm, wv = dim_weights(x32)
    norms, proj = fwht_base(np.asarray(x16, np.float32).astype(np.float64), d)
    norms = f16(norms)
    base = np.asarray(cents, np.float64).reshape(4, D) / ts0
    best = {k: [1.0, ts0, 1e30, 1e30] for k in ("f", "m", "v")}
    deltas = [-0.03, -0.02, -0.01, 0.0, 0.01, 0.02, 0.03, 0.04]
    x32 = np.asarray(x32, np.float64)
    for phase in range(4):
        c = best[{1: "f", 2: "m", 3: "v"}.get(phase, "f")]
        ac, mc = (c[0], c[1] / ts0) if phase else (1.0, 1.0)
        for ia in range(8):
            for it in range(8):
                a = 0.80 + 0.05 * ia if phase == 0 else ac + deltas[ia]
                m = 0.80 + 0.05 * it if phase == 0 else mc + deltas[it]
                ts = ts0 * m
                if vq is None:
                    rec = roundtrip_k(proj, norms, f16(base * ts), rp, d, a)
                else:
                    rec = roundtrip_v(proj, norms, cents, vq, rp, d, a)
                sq = (x32 - rec) ** 2
                e = {"f": sq.mean(), "m": (sq * wm).sum() / len(sq), "v": (sq * wv).sum() / len(sq)}
                me = np.sqrt(sq.max())
                for k in ("f", "m", "v"):
                    if e[k] < best[k][2]:
                        best[k] = [a, ts, e[k], me]
    w = best["f"]
    for k in ("m", "v"):
        if best[k][3] < w[3]:
            w = best[k]
    return w[1], w[0]


# ------------------------------------------------------------------ SmartVQ
# The reference's SmartVQ trainer (ref:src/csrc/qmv_sm75_kernel.cu:2089-2600
# kernels and schedule, :4434-4596 driver), restated in float64: a straight-
# through VQ (hard nearest codeword forward, softmax(-dist / temp) weights
# backward), a rank-8 output transform W = I + A B, Adam with bias correction,
# best-state tracking, patience 15 with rate halving and warm restarts, three
# seeds with an attention-MSE proxy tournament.

def invrotate(x, rp):
    """dst[n][4p + c] = sum_k src[n][4p + k] rp[16p + 4c + k] (.cu:2159-2172)."""
    r = np.asarray(rp, np.float64).reshape(NP, 4, 4)
    return np.einsum("npk,pck->npc", np.asarray(x, np.float64).reshape(-1, NP, 4), r).reshape(-1, D)


def svq_noise(base, seed, scale):
    """base + N(0, 1) scale, one Box-Muller draw per entry from a xorshift
    stream seeded with seed ^ (i 747796405 + 2891336453) (.cu:2387-2401)."""
    base = np.asarray(base, np.float64).ravel()
    i = np.arange(base.size, dtype=np.uint64)
    s = (np.uint64(seed) ^ ((i * np.uint64(747796405) + np.uint64(2891336453)) & np.uint64(0xFFFFFFFF)))
    s = s & np.uint64(0xFFFFFFFF)

    def xs(s):
        s = (s ^ (s << np.uint64(13))) & np.uint64(0xFFFFFFFF)
        s = s ^ (s >> np.uint64(17))
        return (s ^ (s << np.uint64(5))) & np.uint64(0xFFFFFFFF)

    s = xs(s)
    u1 = (s & np.uint64(0xFFFFFF)).astype(np.float64) / 16777216.0 + 1e-7
    s = xs(s)
    u2 = (s & np.uint64(0xFFFFFF)).astype(np.float64) / 16777216.0
    return base + np.sqrt(-2.0 * np.log(u1)) * np.cos(6.2831853 * u2) * scale


def svq_schedule(i, total, lr, lr_mult=1.0):
    """Temperature 1.5 -> 0.1 geometric over steps 0 .. total - 1 and the
    codebook rate, decaying linearly to a floor of 10 % (.cu:2478-2482)."""
    max_it = max(1, total - 1)
    temp = 1.5 * np.exp((np.log(0.1) - np.log(1.5)) * i / max_it)
    return temp, lr * max(0.1, 1.0 - i / total) * lr_mult


def svq_pass(v, attn, cb, wa, wb, rp, T, H_q, H_kv, temp, grad=True, extras=False):
    """One forward (+ backward) pass (.cu:2436-2530).  v f [N][256], attn
    [H_q][T][T] or None, cb [64][256][3], wa [256][8], wb [8][256].  Returns
    (recon loss, dict loss, gcb, gwa, gwb) (gradients None without grad), and
    with extras a dict of the intermediates (rot, idx, recf, grec, gq)."""
    v = np.asarray(v, np.float64)
    cb = np.asarray(cb, np.float64).reshape(NP, 256, 3)
    wa = np.asarray(wa, np.float64).reshape(D, 8)
    wb = np.asarray(wb, np.float64).reshape(8, D)
    N = v.shape[0]
    rot = rotate(v, rp).reshape(N, NP, 4)
    v3 = rot[:, :, :3]
    dist = ((v3[:, :, None, :] - cb[None]) ** 2).sum(-1)  # [N][64][256]
    idx = dist.argmin(-1)  # first minimum
    rec = rot.copy()
    rec[:, :, :3] = np.take_along_axis(cb[None], idx[:, :, None, None].repeat(3, -1), 2)[:, :, 0]
    dict_loss = np.take_along_axis(dist, idx[..., None], -1).sum() / (N * NP * 3)
    # dim 3: round half to even of rot * 16, / 16 (.cu:2139-2155)
    rec[:, :, 3] = np.rint(rot[:, :, 3] * 16.0) / 16.0
    recf = invrotate(rec, rp)
    if attn is not None:
        attn = np.asarray(attn, np.float64)
        n_rep = H_q // H_kv
        dlt = recf + (recf @ wa) @ wb - v
        y = np.stack([attn[h] @ dlt[(h // n_rep) * T:(h // n_rep + 1) * T] for h in range(H_q)])
        recon = (y ** 2).mean()
    else:
        recon = ((recf - v) ** 2).mean()
    if not grad:
        return recon, dict_loss, None, None, None
    if attn is not None:
        g = 2.0 / y.size
        gdl = np.zeros_like(dlt)
        for h in range(H_q):
            kv = h // n_rep
            gdl[kv * T:(kv + 1) * T] += g * attn[h].T @ y[h]
        grec = gdl + (gdl @ wb.T) @ wa.T
        gW = recf.T @ gdl
        gwa, gwb = gW @ wb.T, wa.T @ gW
    else:
        grec = 2.0 * (recf - v) / recf.size
        gwa, gwb = np.zeros_like(wa), np.zeros_like(wb)
    # rotation backward over the first three rotated dims only (the
    # reference drops d = 3, .cu:2300-2314)
    r = np.asarray(rp, np.float64).reshape(NP, 4, 4)
    gq = np.einsum("npd,pdc->npc", grec.reshape(N, NP, 4)[:, :, :3], r[:, :3, :3])
    z = -dist / temp
    w = np.exp(z - z.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    gk = np.einsum("npc,pkc->npk", gq, cb)  # gq . c_k
    swg = (w * gk).sum(-1)
    gd = -(w * (gk - swg[..., None])) / temp
    gcb = np.einsum("npk,npc->pkc", w, gq) + 2.0 * np.einsum(
        "npk,npkc->pkc", gd, cb[None] - v3[:, :, None, :])
    dn = 2.0 / (N * NP * 3)
    hard = np.zeros_like(dist)
    np.put_along_axis(hard, idx[..., None], 1.0, -1)
    gcb += dn * np.einsum("npk,npkc->pkc", hard, cb[None] - v3[:, :, None, :])
    if extras:
        return recon, dict_loss, gcb, gwa, gwb, dict(rot=rot, idx=idx, recf=recf, grec=grec, gq=gq)
    return recon, dict_loss, gcb, gwa, gwb


def _adam(p, g, m, s, lr, bc1, bc2):
    m[:] = 0.9 * m + 0.1 * g
    s[:] = 0.999 * s + 0.001 * g * g
    p -= lr * (m / bc1) / (np.sqrt(s / bc2) + 1e-8)


def svq_train(v, attn, init_cb, rp, T, H_q, H_kv, iterations, n_seeds, lr):
    """The trainer (.cu:4434-4596): returns (codebook [64][256][3], W)."""
    n_seeds = max(1, min(3, n_seeds))
    seeds = [42, 137, 271]
    st = []
    for sd in seeds[:n_seeds]:
        s = dict(cb=np.asarray(init_cb, np.float64).reshape(NP, 256, 3).copy(),
                 wa=svq_noise(np.zeros(2048), (sd * 2654435761 + 1) & 0xFFFFFFFF, 1.0 / 16.0).reshape(D, 8),
                 wb=np.zeros((8, D)), step=0, lr_mult=1.0, stagnant=0, seed=sd)
        for k in ("cb", "wa", "wb"):
            s["m" + k], s["v" + k] = np.zeros_like(s[k]), np.zeros_like(s[k])
        l0, l1, *_ = svq_pass(v, attn, s["cb"], s["wa"], s["wb"], rp, T, H_q, H_kv, 1.5, False)
        s["best"] = l0 + l1
        s["bcb"], s["bwa"], s["bwb"] = s["cb"].copy(), s["wa"].copy(), s["wb"].copy()
        st.append(s)

    def run(s, iters, start):
        total = start + iters
        max_it = max(1, total - 1)
        for i in range(start, total):
            temp, cur = svq_schedule(i, total, lr, s["lr_mult"])
            l0, l1, gcb, gwa, gwb = svq_pass(v, attn, s["cb"], s["wa"], s["wb"], rp, T, H_q, H_kv, temp)
            s["step"] += 1
            bc1, bc2 = 1.0 - 0.9 ** s["step"], 1.0 - 0.999 ** s["step"]
            _adam(s["cb"], gcb, s["mcb"], s["vcb"], cur, bc1, bc2)
            _adam(s["wa"], gwa, s["mwa"], s["vwa"], cur * 0.05, bc1, bc2)
            _adam(s["wb"], gwb, s["mwb"], s["vwb"], cur * 0.05, bc1, bc2)
            loss = l0 + l1  # this step's forward, before the update
            if loss < s["best"] - 1e-7:
                s["best"] = loss
                s["bcb"], s["bwa"], s["bwb"] = s["cb"].copy(), s["wa"].copy(), s["wb"].copy()
                s["stagnant"] = 0
            else:
                s["stagnant"] += 1
            if s["stagnant"] >= 15:
                if s["lr_mult"] > 0.1:
                    s["lr_mult"] *= 0.5
                else:
                    s["lr_mult"] = 3.0
                    ns = 1e-3 * np.exp(np.log(0.01) * i / max_it)
                    s["cb"] = svq_noise(s["bcb"], (s["seed"] ^ i) & 0xFFFFFFFF, ns).reshape(NP, 256, 3)
                    s["wa"], s["wb"] = s["bwa"].copy(), s["bwb"].copy()
                s["stagnant"] = 0

    def proxy(s):
        l0, *_ = svq_pass(v, attn, s["cb"], s["wa"], s["wb"], rp, T, H_q, H_kv, 0.05, False)
        return l0

    r1 = min(iterations, 30)
    r2 = iterations - r1
    prox = []
    for s in st:
        run(s, r1, 0)
        s["cb"], s["wa"], s["wb"] = s["bcb"].copy(), s["bwa"].copy(), s["bwb"].copy()
        prox.append(proxy(s))
    order = sorted(range(n_seeds), key=lambda i: prox[i])
    if r2 > 0:
        for k in order:
            run(st[k], r2, r1)
            prox[k] = proxy(st[k])
    win = order[0]
    for k in order:
        if prox[k] < prox[win]:
            win = k
    w = st[win]
    return w["bcb"], np.eye(D) + w["bwa"] @ w["bwb"]
