"""KHQ calibration driver: KHQD / KHQA dumps -> KHQK v2 centroid file.

The host side of ref:src/khq/calib.mojo:285-566 (main): per dumped layer,
the K path (FWHT base -> K-static centroids -> SmartK tournament over alpha
and the threshold scale) and the V path (FWHT base -> PCA rotors -> per-dim
k-means centroids -> VQ k-means -> 3 Procrustes-Lloyd rotor refinements ->
final centroids and VQ -> attention-aware SmartVQ training -> SmartV
tournament), then one KHQK v2 layer block.  Every step runs on the GPU
through launch_cal_op / launch_cal_svq_train (include/khq.h); this module
only moves data and sequences the calls, as the reference's Mojo driver does.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from . import _lib
from . import centroids as C
from . import dump

D = 256
NP = 64
TOURN_ROWS = 4096   # tournament subset, ref calib.mojo:104
SVQ_ITERS = 100     # ref calib.mojo:177
SVQ_LR = 0.002


class CalibrationError(RuntimeError):
    pass


def _p(t):
    return None if t is None else t.data_ptr()


def cal_op(op, a=None, b=None, c=None, d=None, e=None, f=None, g=None, f1=0.0, f2=0.0,
           i1=0, i2=0, i3=0, i4=0, stream=None):
    """launch_cal_op on torch f32 device tensors (raises on a nonzero code)."""
    rc = _lib.lib().launch_cal_op(op, _p(a), _p(b), _p(c), _p(d), _p(e), _p(f), _p(g), f1, f2,
                                  i1, i2, i3, i4, _lib.stream_handle(stream))
    if rc:
        raise _lib.KhqError(f"launch_cal_op({op})", rc)


def svq_train(v, attn, init_cb, rp, out_cb, *, N, T, H_q, H_kv, iterations=SVQ_ITERS,
              n_seeds=None, lr=SVQ_LR, out_wtrm=None, stream=None):
    """launch_cal_svq_train (the SmartVQ tournament)."""
    if n_seeds is None:
        n_seeds = 3 if attn is not None else 1
    rc = _lib.lib().launch_cal_svq_train(_p(v), _p(attn), _p(init_cb), _p(rp), _p(out_cb),
                                         _p(out_wtrm), N, T, H_q, H_kv, iterations, n_seeds, lr,
                                         _lib.stream_handle(stream))
    if rc:
        raise _lib.KhqError("launch_cal_svq_train", rc)


def svq_pass(v, attn, cb, wa, wb, rp, out_grad, out_loss, *, N, T, H_q, H_kv, temp,
             stream=None):
    """launch_cal_svq_pass: one SmartVQ forward + backward (for tests)."""
    rc = _lib.lib().launch_cal_svq_pass(_p(v), _p(attn), _p(cb), _p(wa), _p(wb), _p(rp),
                                        _p(out_grad), _p(out_loss), N, T, H_q, H_kv, temp,
                                        _lib.stream_handle(stream))
    if rc:
        raise _lib.KhqError("launch_cal_svq_pass", rc)


def calibrate_layer(layer_id: int, k: np.ndarray, v: np.ndarray, attn: np.ndarray | None,
                    *, device="cuda", iterations=SVQ_ITERS, log=print) -> C.LayerCentroids:
    """One layer from its dumped rows k, v f32 [n_tokens][H_kv * 256] and the
    optional attention scores f32 [H_q][n_tokens][n_tokens]."""
    n, dim = k.shape
    heads = dim // D
    rows = n * heads
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)
    new = lambda *s: torch.empty(s, device=device, dtype=torch.float32)
    # (rows, 256) with the heads folded into rows, token-major as the reference
    k32 = f32(k.reshape(rows, D))
    v32 = f32(v.reshape(rows, D))
    k16 = k32.half().float()
    v16 = v32.half().float()
    subm = min(rows, TOURN_ROWS)

    # ---- K
    dk = f32(C.make_d(layer_id))
    rpk = f32(C.identity_rotors())
    normk, projk = new(rows), new(rows, D)
    cal_op(1, a=k32, b=dk, e=normk, f=projk, i1=rows)
    cents_k, tsk = new(4, D), new(1)
    cal_op(2, a=projk, f=cents_k, g=tsk, i1=rows)
    ts_k0 = float(tsk.item())
    log(f"   K static: ts={ts_k0:.6g}")
    cents_k2, tsa_k = new(4, D), new(2)
    cal_op(8, a=k32[:subm].contiguous(), b=k16[:subm].contiguous(), c=dk, d=rpk, e=cents_k,
           f=cents_k2, g=tsa_k, f1=ts_k0, i1=subm)
    ts_k, alpha_k = (float(x) for x in tsa_k.cpu().numpy())

    # ---- V
    dv = f32(C.make_d_v(layer_id))
    vnorm, vbase = new(rows), new(rows, D)
    cal_op(1, a=v32, b=dv, e=vnorm, f=vbase, i1=rows)
    rpv = new(NP, 16)
    cal_op(4, a=vbase, e=rpv, i1=rows)
    cents_v = new(4, D)
    cal_op(5, a=vbase, e=cents_v, i1=rows)
    rot = new(rows, D)
    cal_op(3, a=vbase, b=rpv, e=rot, i1=rows)
    vq = new(NP, 256, 3)
    seed = layer_id * 7919 + 13
    cal_op(6, a=rot, e=vq, i1=rows, i2=seed)
    cal_op(7, a=vbase, b=vq, e=rpv, i1=rows, i2=3)
    cal_op(3, a=vbase, b=rpv, e=rot, i1=rows)
    cal_op(5, a=rot, e=cents_v, i1=rows)
    cal_op(6, a=rot, e=vq, i1=rows, i2=seed)
    vhm = new(rows, D)
    cal_op(10, a=vbase, e=vhm, i1=n, i2=heads)
    if attn is not None:
        if attn.shape[1] != n:
            # a silent fallback to the reconstruction loss would change the result
            raise CalibrationError(f"attn_{layer_id}.bin has {attn.shape[1]} tokens, the dump "
                                   f"has {n}")
        log(f"   [SmartVQ] attention-aware (H_q={attn.shape[0]})")
        svq_train(vhm, f32(attn), vq, rpv, vq, N=rows, T=n, H_q=attn.shape[0], H_kv=heads,
                  iterations=iterations)
    else:
        svq_train(vhm, None, vq, rpv, vq, N=rows, T=n, H_q=heads, H_kv=heads,
                  iterations=iterations)
    tsa_v = new(2)
    cal_op(9, a=v32[:subm].contiguous(), b=v16[:subm].contiguous(), c=dv, d=rpv, e=cents_v,
           f=vq, g=tsa_v, f1=1.95, i1=subm)
    ts_v, alpha_v = (float(x) for x in tsa_v.cpu().numpy())
    log(f"   K: alpha={alpha_k:.4g} ts={ts_k:.6g}   V: alpha={alpha_v:.4g} ts={ts_v:.6g}")
    return C.LayerCentroids(
        layer_id=layer_id, ts_k=ts_k, alpha_k=alpha_k, d_k=dk.cpu().numpy(),
        cents_k=cents_k2.cpu().numpy(), rotor_k=rpk.cpu().numpy(), ts_v=ts_v, alpha_v=alpha_v,
        d_v=dv.cpu().numpy(), cents_v=cents_v.cpu().numpy(), rotor_v=rpv.cpu().numpy(),
        vq=vq.cpu().numpy())


def calibrate(dump_dir: str, out_path: str, *, device="cuda", iterations=SVQ_ITERS,
              log=print) -> list[C.LayerCentroids]:
    """<dump_dir>/kv_dump.bin (+ attn_<layer>.bin when present) -> out_path
    (KHQK v2).  Rejects the dumps the reference rejects (ref calib.mojo:
    400-470): bad magic, dim not a multiple of 256, 0 or > 256 layers, a
    truncated file, layer ids outside [0, 256)."""
    try:
        layers = dump.read_kv_dump(os.path.join(dump_dir, "kv_dump.bin"))
    except ValueError as e:
        raise CalibrationError(str(e)) from e
    out = []
    for layer_id, (k, v) in layers.items():
        dim = k.shape[1]
        if dim < D or dim % D != 0 or not 0 <= layer_id < 256 or len(layers) > 256:
            raise CalibrationError(f"unsupported dump: dim={dim} layer={layer_id}")
        log(f"-- layer {layer_id} tokens={k.shape[0]} rows={k.shape[0] * dim // D}")
        ap = os.path.join(dump_dir, f"attn_{layer_id}.bin")
        attn = dump.attn_matrix(ap) if os.path.exists(ap) else None
        out.append(calibrate_layer(layer_id, k, v, attn, device=device, iterations=iterations,
                                   log=log))
    C.write(out_path, out)
    return out
