"""khq_attn_step_noalloc_fp16 (partials in the library's fixed device array)
against khq_attn_step_fp16 (growable workspace), through the C ABI: two calls
in a row, the second smaller, each identical to the allocating entry point's
output (same kernels, same partition), plus the size guard."""
import numpy as np
import pytest
import torch

from khq import _lib, ops
from khqdata import D, H_KV, H_Q, SCALE, layer_consts, random_rows_np

pytestmark = pytest.mark.gpu


def _case(c_len, win_len, seed, device):
    lc, h = layer_consts(layer_id=seed % 16)
    rows = random_rows_np(max(c_len, 1) * H_KV, seed=seed)
    pay = ops.Payload(max(c_len, 1) * H_KV, device)
    pay.kmask.copy_(torch.from_numpy(rows["kmask"].view(np.int32)))
    for k in ("kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm"):
        getattr(pay, k).copy_(torch.from_numpy(rows[k]))
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal((H_Q, 2 * D)).astype(np.float16)).to(device)
    ring_k = torch.from_numpy(rng.standard_normal((256, H_KV, D)).astype(np.float16)).to(device)
    ring_v = torch.from_numpy(rng.standard_normal((256, H_KV, D)).astype(np.float16)).to(device)
    return dict(q=q, pay=pay, cents=ops.Centroids(lc, device), ring_k=ring_k, ring_v=ring_v,
                c_len=c_len, win_start=c_len % 256, win_len=win_len)


def _run(c, noalloc, device):
    out = torch.full((H_Q, D), float("nan"), device=device, dtype=torch.float16)
    ops.attn_step(c["q"], c["pay"], c["cents"], c["ring_k"], c["ring_v"], out, H_q=H_Q,
                  H_kv=H_KV, c_len=c["c_len"], win_start=c["win_start"],
                  win_len=c["win_len"], ring_cap=256, scale=SCALE, noalloc=noalloc)
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_allocating_entry(device):
    big = _case(32640, 128, seed=3, device=device)
    small = _case(384, 128, seed=4, device=device)
    for c in (big, small):  # two calls in a row, the second smaller
        print(f"noalloc step c_len={c['c_len']} win_len={c['win_len']}", flush=True)
        got = _run(c, True, device)
        want = _run(c, False, device)
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got, want)
    # the array keeps the last call's contents: a repeat of the big case after
    # the small one is still exact
    assert torch.equal(_run(big, True, device), _run(big, False, device))


def test_noalloc_window_only_and_compressed_only(device):
    for c_len, win in ((0, 200), (1000, 0)):
        c = _case(c_len, win, seed=5 + c_len, device=device)
        assert torch.equal(_run(c, True, device), _run(c, False, device))


def test_noalloc_rejects_partials_beyond_the_array(device):
    # H_q 32 / H_kv 4 (portable path): 256 compressed parts + 64 window parts
    # of 32 x 258 floats = 10.6 MB > 8 MiB; refused before any launch
    rc = _lib.call("khq_attn_step_noalloc_fp16", *([None] * 19), 32, 4, 9000, 0, 300, 512,
                   SCALE, 1.0, 1.0, 1e7, None, check=False)
    assert rc == -103
