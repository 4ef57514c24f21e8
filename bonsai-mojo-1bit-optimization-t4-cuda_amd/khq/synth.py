"""Seeded synthetic KHQ states for the benchmark and the parity tests.

Two kinds of compressed rows:
  * random_rows(): uniform-random packed codes (the long-context benchmark
    input): per row an outlier count ~ U[0, 50] of code-3 dims at random
    positions, the other dims uniform over {0, 1, 2}; uniform nibbles and sign
    bits; c_base_mult word uniform in [100, 10000]; norms ~ U(0.5, 2); small
    positive residual scales; uniform 12-bit V fields and VQ high bits.
  * compressed_rows(): the library's own compression of N(0,1) K/V rows
    (what a decode run produces; ~11% outlier dims per K row).
Everything is generated with torch on the requested device from a seed.
"""
from __future__ import annotations

import math

import torch

from .ops import D

ROPE_THETA = 1e7
ROT_DIM = 64


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _uniform(shape, lo, hi, g, device, dtype=torch.float32):
    return (torch.rand(shape, generator=g, device=device) * (hi - lo) + lo).to(dtype)


def random_rows(rows: int, seed: int = 1234, device="cuda") -> dict:
    """Uniform-random packed rows (220 B each) on `device`."""
    g = _gen(seed, device)
    dev = torch.device(device)
    # ---- K mask: n_out ~ U[0, 50] code-3 dims at random positions
    n_out = torch.randint(0, 51, (rows, 1), generator=g, device=dev)
    keys = torch.rand((rows, D), generator=g, device=dev)
    rank = keys.argsort(dim=1).argsort(dim=1)
    codes = torch.randint(0, 3, (rows, D), generator=g, device=dev)
    codes = torch.where(rank < n_out, torch.full_like(codes, 3), codes)
    shifts = (2 * torch.arange(16, device=dev)).view(1, 1, 16)
    words = (codes.view(rows, 16, 16).to(torch.int64) << shifts).sum(dim=2)
    kmask = words.to(torch.int64).bitwise_and(0xFFFFFFFF)
    kmask = torch.where(kmask >= 2 ** 31, kmask - 2 ** 32, kmask).to(torch.int32)
    # ---- K payload
    kpay = torch.randint(0, 256, (rows, 40), generator=g, device=dev, dtype=torch.int64)
    mult = torch.randint(100, 10001, (rows,), generator=g, device=dev, dtype=torch.int64)
    for b in range(4):
        kpay[:, b] = (mult >> (8 * b)) & 0xFF
    kpay[:, 36] = 0x02
    kpay[:, 37:40] = 0
    kpay = kpay.to(torch.uint8)
    knorm = _uniform((rows,), 0.5, 2.0, g, dev, torch.float16)
    krn = _uniform((rows,), 0.002, 0.008, g, dev, torch.float16)
    # ---- V
    vpay = torch.randint(0, 256, (rows, 104), generator=g, device=dev,
                         dtype=torch.int64).to(torch.uint8)
    vnorm = _uniform((rows,), 0.5, 2.0, g, dev, torch.float16)
    vrn = _uniform((rows,), 0.8, 1.2, g, dev, torch.float16)
    vsm = _uniform((rows,), 0.01, 0.05, g, dev, torch.float32).view(torch.uint8).view(rows, 4)
    return {"kmask": kmask, "kpay": kpay, "knorm": knorm, "krn": krn, "vpay": vpay,
            "vnorm": vnorm, "vrn": vrn, "vsm": vsm.contiguous()}


def compressed_rows(pay, cents, seed: int = 1234, chunk: int = 32768) -> None:
    """Fills every row of `pay` (row = token * H_kv + head) with the library's
    own compression of N(0,1) fp16 K and V rows (what a decode run's cache
    holds), seeded, chunk rows at a time on the payload's device."""
    from . import ops

    g = _gen(seed, pay.kmask.device)
    for r0 in range(0, pay.rows, chunk):
        n = min(chunk, pay.rows - r0)
        xk = torch.randn((n, D), generator=g, device=pay.kmask.device).to(torch.float16)
        ops.compress(xk, cents, pay, r0, is_v=False)
        xv = torch.randn((n, D), generator=g, device=pay.kmask.device).to(torch.float16)
        ops.compress(xv, cents, pay, r0, is_v=True)


def rope_halfsplit(x: torch.Tensor, positions: torch.Tensor, rot: int = ROT_DIM,
                   theta: float = ROPE_THETA) -> torch.Tensor:
    """Half-split partial RoPE in fp32 (pairs (i, i+rot/2), freq theta^(-2i/rot))
    on the last dim of x [..., T, H, D] with positions [T]."""
    half = rot // 2
    i = torch.arange(half, device=x.device, dtype=torch.float32)
    freq = torch.exp(math.log(theta) * (-2.0 * i / rot))
    ang = positions.to(torch.float32).view(-1, 1) * freq.view(1, -1)  # [T, half]
    c = torch.cos(ang).unsqueeze(1)
    s = torch.sin(ang).unsqueeze(1)
    xf = x.to(torch.float32)
    x0, x1 = xf[..., :half], xf[..., half:rot]
    out = xf.clone()
    out[..., :half] = x0 * c - x1 * s
    out[..., half:rot] = x0 * s + x1 * c
    return out


def tokens(n: int, H_kv: int, seed: int, device="cuda", start_pos: int = 0) -> dict:
    """N(0,1) fp16 K (unroped), its RoPE'd copy at positions start_pos.., and V."""
    g = _gen(seed, device)
    k = torch.randn((n, H_kv, D), generator=g, device=device).to(torch.float16)
    v = torch.randn((n, H_kv, D), generator=g, device=device).to(torch.float16)
    pos = torch.arange(start_pos, start_pos + n, device=device)
    k_roped = rope_halfsplit(k, pos).to(torch.float16)
    return {"k": k, "k_roped": k_roped, "v": v}


def q_gate(H_q: int, seed: int, device="cuda") -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randn((H_q, 2 * D), generator=g, device=device).to(torch.float16)
