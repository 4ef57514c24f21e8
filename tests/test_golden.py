"""Regression fixtures (tests/golden, written by tests/golden/make_golden.py
from the pinned CPU oracle; the reference ships none of its own).

CPU: the KHKQ v2 reader returns the constants the generator makes, and the
oracle still produces the stored packed rows and decode output bit for bit.
GPU: the compressor reproduces the stored rows bit for bit; the fused decode
step matches the stored output within max-abs 2e-3 / rel 1e-3.
"""
import os

import numpy as np
import pytest

import oracle
from khq import centroids as C
from khqdata import H_KV, H_Q, SCALE, compress_rows, oracle_attn, oracle_window

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden():
    g = np.load(os.path.join(HERE, "golden.npz"))
    lc = C.read(os.path.join(HERE, "layer3.khkq"))[3]
    return g, lc


def _state(g, lc):
    ws, wl = int(g["st_win_start"]), int(g["st_win_len"])
    ring_k = np.zeros((256, H_KV, 256), np.float16)
    ring_v = np.zeros((256, H_KV, 256), np.float16)
    ring_k[ws:ws + wl] = g["st_win_k"]
    ring_v[ws:ws + wl] = g["st_win_v"]
    rows = {k: g["st_" + k] for k in ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm")}
    return dict(lc=lc, h=lc.fp16(), rows=rows, ring_k=ring_k, ring_v=ring_v, q_gate=g["st_q"],
                c_len=int(g["st_c_len"]), win_start=ws, win_len=wl)


def test_khkq_fixture_matches_generator():
    _, lc = _golden()
    want = C.synthetic_layer(3, seed=1234).fp16()
    got = lc.fp16()
    assert set(got) == set(want)
    for k in want:
        assert np.array_equal(got[k].view(np.uint16), want[k].view(np.uint16)), k


def test_oracle_reproduces_golden():
    g, lc = _golden()
    h = lc.fp16()
    kmask, knorm, krn, kpay, ksm = compress_rows(g["xk"], h, False)
    _, vnorm, vrn, vpay, vsm = compress_rows(g["xv"], h, True)
    for name, a in (("kmask", kmask), ("kpay", kpay), ("ksm", ksm), ("vpay", vpay), ("vsm", vsm)):
        assert np.array_equal(a, g[name]), name
    for name, a in (("knorm", knorm), ("krn", krn), ("vnorm", vnorm), ("vrn", vrn)):
        assert np.array_equal(a.view(np.uint16), g[name].view(np.uint16)), name
    st = _state(g, lc)
    _, wc, _ = oracle_attn(st)
    _, ww = oracle_window(st)
    _, out = oracle.merge_gate(wc, ww, st["q_gate"], H_q=H_Q, has_w=True)
    assert np.array_equal(np.asarray(out).view(np.uint16), g["step_out"].view(np.uint16))


@pytest.mark.gpu
def test_gpu_matches_golden(device):
    import torch

    from khq import ops
    from test_gpu_parity import close, payload_from_rows, t

    g, lc = _golden()
    cents = ops.Centroids(lc, device)
    n = g["xk"].shape[0] * H_KV
    pay = ops.Payload(n, device)
    ops.compress(t(g["xk"].reshape(n, 256)), cents, pay, 0, is_v=False)
    ops.compress(t(g["xv"].reshape(n, 256)), cents, pay, 0, is_v=True)
    torch.cuda.synchronize()
    c = lambda a: a.cpu().numpy()
    assert np.array_equal(c(pay.kmask).view(np.uint32), g["kmask"])
    assert np.array_equal(c(pay.kpay), g["kpay"])
    assert np.array_equal(c(pay.vpay), g["vpay"])
    assert np.array_equal(c(pay.vsm), g["vsm"])
    for name in ("knorm", "krn", "vnorm", "vrn"):
        assert np.array_equal(c(getattr(pay, name)).view(np.uint16), g[name].view(np.uint16)), name
    st = _state(g, lc)
    r = st["rows"]
    spay = payload_from_rows(r, r["kmask"].shape[0], device)
    out = torch.zeros((H_Q, 256), device=device, dtype=torch.float16)
    ops.attn_step(t(st["q_gate"]), spay, cents, t(st["ring_k"]), t(st["ring_v"]), out, H_q=H_Q,
                  H_kv=H_KV, c_len=st["c_len"], win_start=st["win_start"], win_len=st["win_len"],
                  ring_cap=256, scale=SCALE)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), g["step_out"])
