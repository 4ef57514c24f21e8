"""Calibration steps on the GPU (launch_cal_op ops 1-10, launch_cal_svq_train
and the khq.calib driver) against the CPU restatement oracle/calib_ref.py
(itself pinned in tests/test_calib_ref.py) and the properties the
mathematics fixes: orthonormal rotors, Lloyd fixed points, the deploy
validator's checks on the written file, loss decrease of SmartVQ."""
import os

import numpy as np
import pytest
import torch

import calib_ref as R
import npref
from khq import calib, centroids as C, dump

pytestmark = pytest.mark.gpu


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def new(*s):
    return torch.zeros(s, device="cuda", dtype=torch.float32)


def _rows(n, seed, scale=None):
    rng = np.random.default_rng(seed)
    sc = rng.uniform(0.3, 3.0, 256) if scale is None else scale
    return (rng.standard_normal((n, 256)) * sc).astype(np.float32)


def test_op1_op2_op3_op10(device):
    x = _rows(700, 0)
    d = C.make_d(5)
    nrm, base = new(700), new(700, 256)
    calib.cal_op(1, a=T(x), b=T(d), e=nrm, f=base, i1=700)
    wn, wb = R.fwht_base(x, d)
    np.testing.assert_allclose(nrm.cpu().numpy(), wn, rtol=1e-5)
    np.testing.assert_allclose(base.cpu().numpy(), wb, rtol=1e-4, atol=1e-6)
    cents, ts = new(4, 256), new(1)
    calib.cal_op(2, a=base, f=cents, g=ts, i1=700)
    wc, wts = R.k_static(base.cpu().numpy().astype(np.float64))
    assert abs(ts.item() - wts) < 1e-4 * wts
    np.testing.assert_allclose(cents.cpu().numpy(), wc, rtol=1e-4, atol=1e-7)
    rp = C.quaternion_rotors(np.random.default_rng(1))
    rot = new(700, 256)
    calib.cal_op(3, a=base, b=T(rp), e=rot, i1=700)
    np.testing.assert_allclose(rot.cpu().numpy(), R.rotate(base.cpu().numpy(), rp), atol=1e-6)
    hm = new(700, 256)
    calib.cal_op(10, a=base, e=hm, i1=175, i2=4)  # 175 tokens x 4 heads
    want = base.cpu().numpy().reshape(175, 4, 256).transpose(1, 0, 2).reshape(700, 256)
    np.testing.assert_array_equal(hm.cpu().numpy(), want)


def test_op4_pca(device):
    rng = np.random.default_rng(2)
    A = rng.standard_normal((64, 4, 4))
    base = np.einsum("npk,pkc->npc", rng.standard_normal((3000, 64, 4)), A).reshape(-1, 256) * 0.1
    rp = new(64, 16)
    calib.cal_op(4, a=T(base), e=rp, i1=3000)
    got = rp.cpu().numpy().reshape(64, 4, 4)
    want = R.pca_rotors(base.astype(np.float32).astype(np.float64)).reshape(64, 4, 4)
    for p in range(64):
        np.testing.assert_allclose(got[p].T @ got[p], np.eye(4), atol=1e-4)
        # same eigenvectors column by column, up to sign
        np.testing.assert_allclose(np.abs(np.diag(got[p].T @ want[p])), 1.0, atol=1e-3)


def test_op5_kmeans4(device):
    x = _rows(2000, 3)
    c = new(4, 256)
    calib.cal_op(5, a=T(x), e=c, i1=2000)
    np.testing.assert_allclose(c.cpu().numpy(), R.kmeans4(x.astype(np.float64)), rtol=2e-4,
                               atol=2e-5)


def test_op6_op7_vq_and_procrustes(device):
    rng = np.random.default_rng(4)
    centers = rng.standard_normal((64, 256, 3)) * 10
    lab = rng.integers(0, 256, (1200, 64))
    pts = centers[np.arange(64)[None, :], lab] + rng.standard_normal((1200, 64, 3)) * 0.01
    rot = np.concatenate([pts, rng.standard_normal((1200, 64, 1))], 2).reshape(1200, 256)
    vq = new(64, 256, 3)
    calib.cal_op(6, a=T(rot), e=vq, i1=1200, i2=7)
    want = R.kmeans_vq(rot.astype(np.float32).astype(np.float64), seed=7, iters=30)
    np.testing.assert_allclose(vq.cpu().numpy(), want, atol=1e-4)
    # Procrustes-Lloyd from random rotors, 3 iterations, codebooks fitted to
    # the rows themselves (well-conditioned M): orthonormal rotors equal to
    # the restatement's
    base = _rows(1200, 5, scale=np.full(256, 0.2))
    rp0 = C.quaternion_rotors(np.random.default_rng(6))
    vq2 = new(64, 256, 3)
    calib.cal_op(6, a=T(R.rotate(base, rp0)), e=vq2, i1=1200, i2=9)
    rp = T(rp0)
    calib.cal_op(7, a=T(base), b=vq2, e=rp, i1=1200, i2=3)
    got = rp.cpu().numpy()
    want = R.procrustes(base.astype(np.float64), vq2.cpu().numpy(), rp0, iters=3)
    np.testing.assert_allclose(got, want, atol=2e-3)
    Rm = got.reshape(64, 4, 4)
    np.testing.assert_allclose(np.einsum("pki,pkj->pij", Rm, Rm),
                               np.broadcast_to(np.eye(4), (64, 4, 4)), atol=2e-3)


@pytest.mark.parametrize("which", ["k", "v"])
def test_op8_op9_tournaments(device, which):
    x32 = _rows(256, 6)
    x16 = x32.astype(np.float16).astype(np.float32)
    lid = 3
    if which == "k":
        d = C.make_d(lid)
        rp = np.tile(np.eye(4).reshape(16), (64, 1)).astype(np.float32)
        _, proj = R.fwht_base(x32, d)
        cents, ts0 = R.k_static(proj)
        cents_out, g = new(4, 256), new(2)
        calib.cal_op(8, a=T(x32), b=T(x16), c=T(d), d=T(rp), e=T(cents), f=cents_out, g=g,
                     f1=float(ts0), i1=256)
        want = R.tournament(x32, x16, d, rp, cents.astype(np.float32), float(np.float32(ts0)))
        np.testing.assert_allclose(cents_out.cpu().numpy(),
                                   R.f16(cents.astype(np.float32) / np.float32(ts0) * g[0].item()),
                                   rtol=2e-3, atol=1e-6)
    else:
        d = C.make_d_v(lid)
        lc = C.synthetic_layer(lid, alpha_v=1.0 / 16.0)
        rp, cents, vq = lc.rotor_v, lc.cents_v, lc.vq / 16.0
        g = new(2)
        calib.cal_op(9, a=T(x32), b=T(x16), c=T(d), d=T(rp), e=T(cents), f=T(vq), g=g,
                     f1=1.95, i1=256)
        want = R.tournament(x32, x16, d, rp, cents, 1.95, vq=vq)
    ts, alpha = g.cpu().numpy()
    print(f"{which}: gpu ts {ts:.6f} alpha {alpha:.4f}, cpu ts {want[0]:.6f} alpha {want[1]:.4f}")
    assert abs(ts - want[0]) < 1e-4 * want[0] and abs(alpha - want[1]) < 1e-5


def _svq_case(n_tok=96, heads=2, seed=7):
    rng = np.random.default_rng(seed)
    N = n_tok * heads
    v = (rng.standard_normal((N, 256)) * 0.06).astype(np.float32)
    rp = C.quaternion_rotors(rng)
    rot = R.rotate(v, rp)
    init = R.kmeans_vq(rot, seed=11, iters=3).astype(np.float32)
    return v, rp, init, N


def _recon_mse(v, rp, cb):
    rot = R.rotate(v, rp).reshape(-1, 64, 4)
    rec = rot.copy()
    for p in range(64):
        rec[:, p, :3] = cb[p][R.nearest(rot[:, p, :3], cb[p])]
    rec[:, :, 3] = np.rint(rot[:, :, 3] * 16) / 16
    back = np.einsum("npk,pck->npc", rec, np.asarray(rp, np.float64).reshape(64, 4, 4)).reshape(-1, 256)
    return ((back - v) ** 2).mean()


def test_svq_train_reconstruction_mode(device):
    v, rp, init, N = _svq_case()
    out = new(64, 256, 3)
    calib.svq_train(T(v), None, T(init), T(rp), out, N=N, T=96, H_q=2, H_kv=2, iterations=0)
    np.testing.assert_array_equal(out.cpu().numpy(), init)  # no step: the initial codebook
    calib.svq_train(T(v), None, T(init), T(rp), out, N=N, T=96, H_q=2, H_kv=2, iterations=60)
    cb = out.cpu().numpy()
    assert np.all(np.isfinite(cb))
    before, after = _recon_mse(v, rp, init), _recon_mse(v, rp, cb)
    print(f"SmartVQ reconstruction MSE {before:.4e} -> {after:.4e}")
    assert after < before


def test_svq_train_attention_mode(device):
    v, rp, init, N = _svq_case(n_tok=64, heads=2, seed=8)
    rng = np.random.default_rng(9)
    H_q, Tn = 4, 64
    s = rng.standard_normal((H_q, Tn, Tn)) + np.triu(np.full((Tn, Tn), -1e9), 1)[None]
    attn = np.exp(s - s.max(-1, keepdims=True))
    attn = (attn / attn.sum(-1, keepdims=True)).astype(np.float32)
    out, wt = new(64, 256, 3), new(256, 256)
    calib.svq_train(T(v), T(attn), T(init), T(rp), out, N=N, T=Tn, H_q=H_q, H_kv=2,
                    iterations=40, out_wtrm=wt)
    cb, W = out.cpu().numpy(), wt.cpu().numpy()
    assert np.all(np.isfinite(cb)) and np.all(np.isfinite(W))
    assert np.abs(W - np.eye(256)).max() < 0.5  # I + A B with a small rank-8 part
    assert not np.array_equal(cb, init)
    # the winner is no worse than the initial codebook on the plain reconstruction
    assert _recon_mse(v, rp, cb) < 1.05 * _recon_mse(v, rp, init)


def _svq_margin_case(T=32, H_kv=2, H_q=4, seed=21, shift=0.0):
    """Rows whose rotated dims 0..2 sit near one codeword each (offsets well
    inside half the codebook spacing), so the GPU and the float64
    restatement pick the same hard codewords; with shift, the rows of each
    codeword share an offset of that length (training has something to
    improve)."""
    rng = np.random.default_rng(seed)
    N = T * H_kv
    cb = (rng.standard_normal((64, 256, 3)) * 0.06).astype(np.float32)
    rp = C.quaternion_rotors(rng).astype(np.float32)
    k = rng.integers(0, 256, (N, 64))
    off = rng.standard_normal((64, 256, 3))
    off *= shift / np.linalg.norm(off, axis=-1, keepdims=True)
    rot = np.empty((N, 64, 4))
    rot[:, :, :3] = (cb[np.arange(64)[None, :], k] + off[np.arange(64)[None, :], k]
                     + rng.standard_normal((N, 64, 3)) * 2e-4)
    rot[:, :, 3] = rng.standard_normal((N, 64)) * 0.06
    # rot[p][c] = sum_k v[p][k] rp[16 p + 4 k + c]: v = rot M^T for the orthogonal M
    M = rp.astype(np.float64).reshape(64, 4, 4)
    v = np.einsum("npc,pkc->npk", rot, M).reshape(N, 256).astype(np.float32)
    s = rng.standard_normal((H_q, T, T)) + np.triu(np.full((T, T), -1e9), 1)[None]
    attn = np.exp(s - s.max(-1, keepdims=True))
    attn = (attn / attn.sum(-1, keepdims=True)).astype(np.float32)
    return v, rp, cb, attn, N, T, H_q, H_kv


@pytest.mark.parametrize("mode", ["attention", "reconstruction"])
def test_svq_pass_vs_restatement(device, mode):
    """One SmartVQ pass (launch_cal_svq_pass) against the float64
    restatement: losses, the straight-through codebook gradient and the
    transform gradients."""
    v, rp, cb, attn, N, Tn, H_q, H_kv = _svq_margin_case()
    if mode == "reconstruction":
        attn = None
    rng = np.random.default_rng(22)
    wa = (rng.standard_normal((256, 8)) / 16).astype(np.float32)
    wb = (rng.standard_normal((8, 256)) / 64).astype(np.float32)
    g, l = new(49152 + 4096), new(2)
    calib.svq_pass(T(v), None if attn is None else T(attn), T(cb), T(wa), T(wb), T(rp), g, l,
                   N=N, T=Tn, H_q=H_q, H_kv=H_kv, temp=0.3)
    rl, dl, gcb, gwa, gwb = R.svq_pass(v, attn, cb, wa, wb, rp, Tn, H_q, H_kv, 0.3)
    got_l, got = l.cpu().numpy(), g.cpu().numpy()
    np.testing.assert_allclose(got_l, [rl, dl], rtol=1e-4)
    for a, w in ((got[:49152], gcb.ravel()), (got[49152:51200], gwa.ravel()),
                 (got[51200:], gwb.ravel())):
        np.testing.assert_allclose(a, w, rtol=1e-3, atol=1e-4 * max(np.abs(w).max(), 1e-30))


def test_svq_train_vs_restatement(device):
    """The whole trainer (3 seeds, Adam steps, best tracking, the proxy
    tournament) against the float64 restatement; with no rate the output
    is the initial codebook and W = I."""
    v, rp, cb, attn, N, Tn, H_q, H_kv = _svq_margin_case(seed=23, shift=4e-3)
    out, wt = new(64, 256, 3), new(256, 256)
    for it, lr in ((6, 1e-3), (20, 0.0)):
        calib.svq_train(T(v), T(attn), T(cb), T(rp), out, N=N, T=Tn, H_q=H_q, H_kv=H_kv,
                        iterations=it, n_seeds=3, lr=lr, out_wtrm=wt)
        want_cb, want_w = R.svq_train(v, attn, cb, rp, Tn, H_q, H_kv, iterations=it, n_seeds=3,
                                      lr=lr)
        got_cb, got_w = out.cpu().numpy(), wt.cpu().numpy()
        print(f"SmartVQ {it} steps lr {lr}: max |cb - ref| {np.abs(got_cb - want_cb).max():.3e}, "
              f"max |W - ref| {np.abs(got_w - want_w).max():.3e}")
        np.testing.assert_allclose(got_cb, want_cb, atol=max(1e-3 * lr, 1e-7))
        np.testing.assert_allclose(got_w, want_w, atol=max(1e-3 * lr, 1e-7))
        if lr == 0.0:
            np.testing.assert_array_equal(got_cb, cb)
        else:  # the winner's best state moved away from the start
            assert np.abs(want_cb - cb).max() > 0.5 * lr


def _write_attn(path, H_q, n, H_kv, rng):
    with open(path, "wb") as f:
        import struct
        f.write(struct.pack("<IIII", dump.MAGIC_ATTN, H_q, H_kv, 256))
        for t in range(n):
            s = rng.standard_normal((H_q, t + 1))
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            f.write(struct.pack("<I", t + 1))
            f.write(p.astype(np.float16).tobytes())


def test_calibrate_end_to_end(device, tmp_path):
    """Synthetic dumps of two layers -> KHQK v2 file that passes the deploy
    validator, with orthonormal rotors, the K-static centroid pattern, +-1
    d vectors, and a runtime compress / decode round trip close to the input."""
    rng = np.random.default_rng(10)
    n, H_kv, H_q = 160, 4, 8
    scale = rng.uniform(0.3, 2.0, H_kv * 256)
    layers = {}
    for lid in (3, 7):
        k = (rng.standard_normal((n, H_kv * 256)) * scale).astype(np.float32)
        v = (rng.standard_normal((n, H_kv * 256)) * scale[::-1]).astype(np.float32)
        layers[lid] = (k, v)
    dump.write_kv_dump(str(tmp_path / "kv_dump.bin"), layers)
    _write_attn(str(tmp_path / "attn_3.bin"), H_q, n, H_kv, rng)  # layer 7: no scores
    out = str(tmp_path / "cents.bin")
    res = calib.calibrate(str(tmp_path), out, iterations=20, log=lambda *a: None)
    assert [L.layer_id for L in res] == [3, 7]
    assert C.validate(out) == []
    got = C.read(out)
    for lid in (3, 7):
        L = got[lid]
        assert np.all(np.abs(L.d_k) == 1) and np.all(np.abs(L.d_v) == 1)
        np.testing.assert_array_equal(L.d_k, C.make_d(lid))
        np.testing.assert_array_equal(L.d_v, C.make_d_v(lid))
        for rot in (L.rotor_k, L.rotor_v):
            Rm = rot.reshape(64, 4, 4)
            np.testing.assert_allclose(np.einsum("pki,pkj->pij", Rm, Rm),
                                       np.broadcast_to(np.eye(4), (64, 4, 4)), atol=2e-3)
        ck = L.cents_k
        assert np.all(ck[0] == 0) and np.allclose(ck[1], -ck[2]) and np.allclose(ck[3], ck[2])
        assert 0.5 < L.alpha_k < 1.5 and 0.5 < L.alpha_v < 1.5
        # the runtime compressor with these centroids, decoded independently
        from khq import ops
        h = L.fp16()
        k0 = layers[lid][0][:32].reshape(32 * H_kv, 256).astype(np.float16)
        pay = ops.Payload(32 * H_kv)
        cents = ops.Centroids(L)
        ops.compress(torch.from_numpy(k0).cuda(), cents, pay, 0, is_v=False)
        torch.cuda.synchronize()
        kd = npref.decode_k(pay.kmask.cpu().numpy().view(np.uint32), pay.kpay.cpu().numpy(),
                            pay.knorm.cpu().numpy(), pay.krn.cpu().numpy(), h["cents_k"],
                            h["rotor_k"], h["d_k"], L.alpha_k)
        x = k0.astype(np.float64)
        cs = (kd * x).sum(1) / (np.linalg.norm(kd, axis=1) * np.linalg.norm(x, axis=1))
        print(f"layer {lid}: K round trip cos-sim min {cs.min():.3f} mean {cs.mean():.3f}")
        assert cs.min() > 0.85
