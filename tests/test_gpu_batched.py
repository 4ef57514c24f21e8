"""GPU parity of the batched decode step (khq_attn_step_batched_fp16): ragged
sequences in one call, each against the oracle (small cases) or against the
library's own single-sequence step (the 32-sequence ragged configuration,
L ~ U[1024, 16384]).

Bar: attention outputs within max-abs 2e-3 and rel 1e-3 of the oracle; the
single-step comparison uses the same tolerance (the two calls partition the
tokens differently, so their fp32 sums round differently).
"""
import numpy as np
import pytest
import torch

import oracle
from khq import ops, synth
from khqdata import (D, H_KV, H_Q, SCALE, layer_consts, oracle_attn, oracle_window,
                     random_rows_np)
from test_gpu_parity import close, margins, payload_from_rows, t

pytestmark = pytest.mark.gpu


def _seq_state(rng, lc, h, c_len, win_start, win_len, seed):
    rows = random_rows_np(max(c_len, 1) * H_KV, seed=seed)
    ring_k = rng.standard_normal((256, H_KV, D)).astype(np.float16)
    ring_v = rng.standard_normal((256, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((H_Q, 2 * D)).astype(np.float16)
    return dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len, ring_k=ring_k, ring_v=ring_v,
                win_start=win_start, win_len=win_len)


def _oracle_out(st):
    if st["c_len"] == 0:
        _, ww = oracle_window(st)
        return oracle.merge_gate(ww, ww, st["q_gate"], H_q=H_Q, has_w=False)[1]
    _, wc, _ = oracle_attn(st)
    if st["win_len"] == 0:
        return oracle.merge_gate(wc, wc, st["q_gate"], H_q=H_Q, has_w=False)[1]
    _, ww = oracle_window(st)
    return oracle.merge_gate(wc, ww, st["q_gate"], H_q=H_Q, has_w=True)[1]


# (c_len, win_start, win_len): window only, compressed only, wrapped window,
# full ring, a single tile, a ragged tail, long and short sequences together.
CASES = [(0, 0, 200), (2048, 0, 0), (384, 128, 216), (1280, 88, 256), (16, 16, 1), (37, 37, 5),
         (5000, 136, 128), (129, 129, 130)]


@pytest.mark.parametrize("order", ["given", "reversed"])
def test_batched_matches_oracle(device, order):
    lc, h = layer_consts()
    rng = np.random.default_rng(11)
    cases = CASES if order == "given" else CASES[::-1]
    states = [_seq_state(rng, lc, h, c, ws, wl, seed=100 + i)
              for i, (c, ws, wl) in enumerate(cases)]
    cents = ops.Centroids(lc, device)
    seqs = []
    for st in states:
        n_rows = st["rows"]["kmask"].shape[0]
        seqs.append(dict(q_gate=t(st["q_gate"]), pay=payload_from_rows(st["rows"], n_rows),
                         ring_k=t(st["ring_k"]), ring_v=t(st["ring_v"]),
                         out=torch.zeros((H_Q, D), device=device, dtype=torch.float16),
                         c_len=st["c_len"], win_start=st["win_start"], win_len=st["win_len"],
                         ring_cap=256))
    ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    for st, s in zip(states, seqs):
        close(s["out"].cpu().numpy(), _oracle_out(st))


def test_batched_back_to_back_calls(device):
    """Six batched calls queued back to back with no synchronisation between
    them (each stages its arguments in a pinned slot of a four-slot ring that
    the GPU uploads in stream order; the fifth and sixth calls reuse slots)
    give bit for bit the outputs of the same calls made one at a time."""
    lc, h = layer_consts()
    rng = np.random.default_rng(12)
    cents = ops.Centroids(lc, device)
    calls = []
    for k in range(6):
        cases = CASES[k % len(CASES):] + CASES[:k % len(CASES)]
        cases = cases[: 3 + k]
        seqs = []
        for i, (c, ws, wl) in enumerate(cases):
            st = _seq_state(rng, lc, h, c, ws, wl, seed=500 + 10 * k + i)
            n_rows = st["rows"]["kmask"].shape[0]
            seqs.append(dict(q_gate=t(st["q_gate"]), pay=payload_from_rows(st["rows"], n_rows),
                             ring_k=t(st["ring_k"]), ring_v=t(st["ring_v"]),
                             out=torch.zeros((H_Q, D), device=device, dtype=torch.float16),
                             c_len=st["c_len"], win_start=st["win_start"], win_len=st["win_len"],
                             ring_cap=256))
        calls.append(seqs)
    want = []
    for seqs in calls:
        assert ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE) == 0
        torch.cuda.synchronize()
        want.append([s["out"].clone() for s in seqs])
        for s in seqs:
            s["out"].zero_()
    torch.cuda.synchronize()
    for seqs in calls:
        assert ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE) == 0
    torch.cuda.synchronize()
    for k, seqs in enumerate(calls):
        for i, s in enumerate(seqs):
            a = s["out"].cpu().numpy().view(np.uint16)
            b = want[k][i].cpu().numpy().view(np.uint16)
            assert np.array_equal(a, b), (k, i)


def test_batched_error_codes(device):
    lc, _ = layer_consts()
    cents = ops.Centroids(lc, device)
    pay = ops.Payload(64 * H_KV, device)
    z = torch.zeros((H_Q, 2 * D), device=device, dtype=torch.float16)
    rk = torch.zeros((256, H_KV, D), device=device, dtype=torch.float16)
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    base = dict(q_gate=z, pay=pay, ring_k=rk, ring_v=rk, out=out, c_len=64, win_start=0,
                win_len=10, ring_cap=256)
    bad = [dict(base, c_len=0, win_len=0), dict(base, win_len=257), dict(base, c_len=-1)]
    for b in bad:
        assert ops.attn_step_batched([base, b], cents, H_q=H_Q, H_kv=H_KV, scale=SCALE,
                                     check=False) == -100
    assert ops.attn_step_batched([dict(base, c_len=16, win_len=0)], cents, H_q=H_Q, H_kv=5, scale=SCALE,
                                 check=False) == -100


def test_batched_c4_ragged_32(device):
    """32 ragged sequences, L ~ U[1024, 16384] compressed tokens each plus a
    raw window of L % 256 + 1 tokens, against one single-sequence step each;
    then the oracle on the two shortest, a middle and the longest sequence."""
    lc, h = layer_consts()
    rng = np.random.default_rng(44)
    lens = rng.integers(1024, 16385, 32)
    cents = ops.Centroids(lc, device)
    seqs, singles = [], []
    for i, L in enumerate(lens):
        L = int(L)
        rows = synth.random_rows(L * H_KV, seed=500 + i, device=device)
        pay = ops.Payload(L * H_KV, device)
        for k in ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm"):
            getattr(pay, k).copy_(rows[k])
        wl = L % 256 + 1
        s = dict(q_gate=synth.q_gate(H_Q, seed=900 + i, device=device), pay=pay,
                 ring_k=torch.randn((256, H_KV, D), device=device).half(),
                 ring_v=torch.randn((256, H_KV, D), device=device).half(),
                 out=torch.zeros((H_Q, D), device=device, dtype=torch.float16),
                 c_len=L, win_start=L % 256, win_len=wl, ring_cap=256)
        seqs.append(s)
    ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    for s in seqs:
        o = torch.zeros_like(s["out"])
        ops.attn_step(s["q_gate"], s["pay"], cents, s["ring_k"], s["ring_v"], o, H_q=H_Q,
                      H_kv=H_KV, c_len=s["c_len"], win_start=s["win_start"],
                      win_len=s["win_len"], ring_cap=256, scale=SCALE)
        singles.append(o)
    torch.cuda.synchronize()
    for s, o in zip(seqs, singles):
        close(s["out"].float().cpu().numpy(), o.float().cpu().numpy())
    # the batched call is deterministic
    first = [s["out"].clone() for s in seqs]
    ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    assert all(torch.equal(a, s["out"]) for a, s in zip(first, seqs))
    # the oracle directly on the two shortest, a middle and the longest sequence
    order = np.argsort(lens)
    for i in (order[0], order[1], order[len(order) // 2], order[-1]):
        s = seqs[int(i)]
        rows = {k: getattr(s["pay"], k).cpu().numpy() for k in
                ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm")}
        rows["kmask"] = rows["kmask"].view(np.uint32)
        st = dict(rows=rows, h=h, lc=lc, q_gate=s["q_gate"].cpu().numpy(), c_len=s["c_len"],
                  ring_k=s["ring_k"].cpu().numpy(), ring_v=s["ring_v"].cpu().numpy(),
                  win_start=s["win_start"], win_len=s["win_len"])
        want = _oracle_out(st)
        close(s["out"].cpu().numpy(), want)
        # the outputs are fp16: beyond the tolerance, the error of every output
        # of magnitude >= 1e-3 is at most one fp16 unit in the last place of
        # the float64 result (the two sides round near-ties differently); the
        # share of the tolerance is reported
        got16 = s["out"].cpu().numpy()
        big = np.abs(want) >= 1e-3
        ulp = np.spacing(np.abs(want[big]).astype(np.float16)).astype(np.float64)
        ulps = (np.abs(got16.astype(np.float64)[big] - want[big]) / ulp).max()
        m_abs, m_rel = margins(got16, want)
        print(f"C4 sequence of {s['c_len']} + {s['win_len']} tokens: max-abs err / 2e-3 = "
              f"{m_abs:.3f}, rel err / 1e-3 = {m_rel:.3f}, {ulps:.2f} fp16 ulp", flush=True)
        assert ulps <= 1.0, ulps


def test_batched_refuses_graph_capture(device):
    """Under HIP graph capture the batched call returns -105 and launches
    nothing (its argument copy comes from host staging a later call reuses)."""
    lc, h = layer_consts()
    rng = np.random.default_rng(12)
    st = _seq_state(rng, lc, h, 384, 128, 128, seed=300)
    cents = ops.Centroids(lc, device)
    n_rows = st["rows"]["kmask"].shape[0]
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    seqs = [dict(q_gate=t(st["q_gate"]), pay=payload_from_rows(st["rows"], n_rows),
                 ring_k=t(st["ring_k"]), ring_v=t(st["ring_v"]), out=out, c_len=384,
                 win_start=128, win_len=128, ring_cap=256)]
    ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE)  # eager: fine
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=SCALE, check=False)
    assert rc == -105
