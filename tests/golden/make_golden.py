"""Writes the regression fixtures of this directory from the CPU oracle.

The reference ships no KHQ golden vector or unit test, so these are not
reference outputs: they freeze the oracle's results (after its pins in
tests/test_oracle_pins.py pass) on small fixed inputs, so that a later change
to the oracle, the synthetic centroid generator or a GPU kernel shows up as a
bit difference against files that do not move.

  layer3.khkq   one layer of constants in the reference's KHKQ v2 centroid
                file format (written by khq.centroids.write)
  golden.npz    compress inputs / packed outputs (8 tokens x 4 KV heads, K
                and V) and a two-region decode step (64 compressed + 16 raw
                tokens): its packed rows, the window's ring slots, q_gate and
                the gated output

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "bonsai-mojo-1bit-optimization-t4-cuda_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    sys.path.insert(0, p)

import oracle  # noqa: E402
from khq import centroids as C  # noqa: E402
from khqdata import (H_KV, H_Q, compress_rows, oracle_attn, oracle_window,  # noqa: E402
                     two_region_state)


def main():
    lc = C.synthetic_layer(3, seed=1234)
    C.write(os.path.join(HERE, "layer3.khkq"), [lc])
    h = C.read(os.path.join(HERE, "layer3.khkq"))[3].fp16()
    rng = np.random.default_rng(2024)
    xk = rng.standard_normal((8, H_KV, 256)).astype(np.float16)
    xv = rng.standard_normal((8, H_KV, 256)).astype(np.float16)
    kmask, knorm, krn, kpay, ksm = compress_rows(xk, h, False)
    _, vnorm, vrn, vpay, vsm = compress_rows(xv, h, True)
    st = two_region_state(seed=11, n_tokens=80, boundary=64)
    ws, wl = st["win_start"], st["win_len"]
    _, wc, _ = oracle_attn(st)
    _, ww = oracle_window(st)
    _, out = oracle.merge_gate(wc, ww, st["q_gate"], H_q=H_Q, has_w=True)
    r = st["rows"]
    np.savez_compressed(
        os.path.join(HERE, "golden.npz"),
        xk=xk, xv=xv, kmask=kmask, knorm=knorm, krn=krn, kpay=kpay, ksm=ksm,
        vnorm=vnorm, vrn=vrn, vpay=vpay, vsm=vsm,
        st_kmask=r["kmask"], st_kpay=r["kpay"], st_knorm=r["knorm"], st_krn=r["krn"],
        st_vpay=r["vpay"], st_vnorm=r["vnorm"], st_vrn=r["vrn"], st_vsm=r["vsm"],
        st_win_k=st["ring_k"][ws:ws + wl], st_win_v=st["ring_v"][ws:ws + wl], st_q=st["q_gate"],
        st_c_len=st["c_len"], st_win_start=st["win_start"], st_win_len=st["win_len"],
        step_out=out)


if __name__ == "__main__":
    main()
