"""HIP graph capture of the single-sequence step: khq_attn_step_fp16 (after
khq_workspace_reserve) and khq_attn_step_noalloc_fp16 captured once, replayed
several times on new query contents with eager KHQ and torch work between the
replays; every replay equals the eager step on the same inputs bit for bit
(the kernels are deterministic: fixed partition, fixed merge order)."""
import numpy as np
import pytest
import torch

from khq import ops
from khqdata import D, H_KV, H_Q, SCALE, layer_consts, random_rows_np, two_region_state
from test_gpu_parity import _gpu_state, payload_from_rows, t

pytestmark = pytest.mark.gpu


def _cases(device):
    st = two_region_state(seed=51)
    pay, cents = _gpu_state(st)
    small = dict(pay=pay, cents=cents, ring_k=t(st["ring_k"]), ring_v=t(st["ring_v"]),
                 c_len=st["c_len"], win_start=st["win_start"], win_len=st["win_len"])
    lc, _ = layer_consts(layer_id=6)
    c_len = 8192
    rows = random_rows_np(c_len * H_KV, seed=52)
    ring = torch.from_numpy(np.random.default_rng(53).standard_normal((256, H_KV, D))
                            .astype(np.float16)).to(device)
    big = dict(pay=payload_from_rows(rows, c_len * H_KV), cents=ops.Centroids(lc, device),
               ring_k=ring, ring_v=ring, c_len=c_len, win_start=c_len % 256, win_len=128)
    return {"384+128": small, "8192+128": big}


@pytest.mark.parametrize("noalloc", [False, True], ids=["workspace", "noalloc"])
def test_captured_step_replays_match_eager(device, noalloc):
    rng = np.random.default_rng(54)
    ops.workspace_reserve(64 << 20)
    for name, c in _cases(device).items():
        q = torch.empty((H_Q, 2 * D), device=device, dtype=torch.float16)
        q.copy_(torch.from_numpy(rng.standard_normal((H_Q, 2 * D)).astype(np.float16)))
        out_g = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
        out_e = torch.zeros_like(out_g)

        def step(out, check=True):
            return ops.attn_step(q, c["pay"], c["cents"], c["ring_k"], c["ring_v"], out,
                                 H_q=H_Q, H_kv=H_KV, c_len=c["c_len"],
                                 win_start=c["win_start"], win_len=c["win_len"], ring_cap=256,
                                 scale=SCALE, noalloc=noalloc, check=check)

        step(out_g)  # warm-up outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            rc = step(out_g, check=False)
        assert rc == 0, (name, rc)
        for rep in range(4):
            print(f"graph replay {rep} of {name} noalloc={noalloc}", flush=True)
            q.copy_(torch.from_numpy(rng.standard_normal((H_Q, 2 * D)).astype(np.float16)))
            out_g.zero_()
            g.replay()
            torch.cuda.synchronize()
            # eager work between the replays: the same step, and unrelated torch work
            assert step(out_e) == 0
            junk = torch.randn((1 << 20,), device=device).sum()
            torch.cuda.synchronize()
            assert torch.isfinite(junk)
            a = out_g.cpu().numpy().view(np.uint16)
            b = out_e.cpu().numpy().view(np.uint16)
            assert np.array_equal(a, b), (name, rep)
            assert np.isfinite(out_g.float().cpu().numpy()).all()


def test_graph_survives_workspace_growth(device):
    """A graph captured over the shared workspace keeps replaying correctly
    after a later eager call grows the workspace: the captured buffer is
    retired, not freed, so memory torch hands out afterwards (filled with NaN
    here) never aliases it."""
    rng = np.random.default_rng(57)
    c = _cases(device)["8192+128"]
    q = torch.from_numpy(rng.standard_normal((H_Q, 2 * D)).astype(np.float16)).to(device)
    out_g = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    out_e = torch.zeros_like(out_g)

    def step(out, check=True):
        return ops.attn_step(q, c["pay"], c["cents"], c["ring_k"], c["ring_v"], out,
                             H_q=H_Q, H_kv=H_KV, c_len=c["c_len"], win_start=c["win_start"],
                             win_len=c["win_len"], ring_cap=256, scale=SCALE, check=check)

    step(out_g)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert step(out_g, check=False) == 0
    print("graph captured; growing the workspace past every earlier size", flush=True)
    ops.workspace_reserve(768 << 20)
    junk = [torch.full((64 << 20,), float("nan"), device=device) for _ in range(4)]
    torch.cuda.synchronize()
    for rep in range(3):
        out_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert step(out_e) == 0
        torch.cuda.synchronize()
        assert np.array_equal(out_g.cpu().numpy().view(np.uint16),
                              out_e.cpu().numpy().view(np.uint16)), rep
    del junk
