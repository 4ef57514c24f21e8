"""Two streams issuing KHQ steps at once share the library's split workspace
safely: the library orders a launch after the previous user stream's work
(an event handed across), so each stream's outputs equal those of the same
steps run one after another on one stream."""
import numpy as np
import pytest
import torch

from khq import ops, synth
from khq.centroids import synthetic_layer
from khqdata import D, H_KV, H_Q, SCALE

pytestmark = pytest.mark.gpu


def _layer(c_len, seed, device):
    pay = ops.Payload(c_len * H_KV, device)
    for k, v in synth.random_rows(c_len * H_KV, seed=seed, device=device).items():
        getattr(pay, k).copy_(v)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return dict(pay=pay, cents=ops.Centroids(synthetic_layer(seed % 7, seed=1234), device),
                q=synth.q_gate(H_Q, seed=seed + 1, device=device),
                ring_k=torch.randn((256, H_KV, D), generator=g, device=device).half(),
                ring_v=torch.randn((256, H_KV, D), generator=g, device=device).half(),
                c_len=c_len)


def _step(L, out, stream):
    ops.attn_step(L["q"], L["pay"], L["cents"], L["ring_k"], L["ring_v"], out, H_q=H_Q,
                  H_kv=H_KV, c_len=L["c_len"], win_start=L["c_len"] % 256, win_len=128,
                  ring_cap=256, scale=SCALE, stream=stream)


def test_two_streams_share_workspace(device):
    # different context lengths: different partial counts in the shared workspace
    layers = [_layer(8192, 11, device), _layer(2048, 12, device)]
    want = []
    for L in layers:
        o = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
        _step(L, o, torch.cuda.current_stream())
        want.append(o)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.zeros((H_Q, D), device=device, dtype=torch.float16) for _ in range(12)]
            for _ in layers]
    for i in range(12):  # interleaved issue, no host synchronisation in between
        for L, s, o in zip(layers, streams, outs):
            with torch.cuda.stream(s):
                _step(L, o[i], s)
    torch.cuda.synchronize()
    for w, o in zip(want, outs):
        for x in o:
            assert torch.equal(x, w)
