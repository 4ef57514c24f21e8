"""End-to-end KHQ layer runtime on the GPU (ref:src/khq/runtime.mojo:454-613)
against a step-by-step CPU simulation built from the oracle.

Also the reference's integration gates (ref:deploy_on_kaggle.sh:1763-1941)
restated as assertions: compression cadence (event k leaves boundary 128 k
and a 128-token raw window) and the K-norm fingerprint of the compressed rows.
"""
import numpy as np
import pytest
import torch

import oracle
from khq import layer as KL
from khqdata import D, H_KV, H_Q, N_REP, SCALE, THETA, layer_consts, rope_fp16_rows

pytestmark = pytest.mark.gpu

N_STEPS = 520


class Sim:
    """CPU twin of KhqLayer using the oracle for every kernel."""

    def __init__(self, lc, h, splits, cap=4096):
        self.lc, self.h, self.splits, self.cap = lc, h, splits, cap
        self.ring_k = np.zeros((256, H_KV, D), np.float16)
        self.ring_v = np.zeros((256, H_KV, D), np.float16)
        self.ring_u = np.zeros((256, H_KV, D), np.float16)
        rows = cap * H_KV
        self.kmask = np.zeros((rows, 16), np.uint32)
        self.kpay = np.zeros((rows, 40), np.uint8)
        self.vpay = np.zeros((rows, 104), np.uint8)
        self.knorm = np.zeros(rows, np.float16)
        self.krn = np.zeros(rows, np.float16)
        self.vnorm = np.zeros(rows, np.float16)
        self.vrn = np.zeros(rows, np.float16)
        self.vsm = np.zeros((rows, 4), np.uint8)
        self.boundary = 0
        self.write_pos = 0

    def step(self, q_gate, k_roped, v, k_unroped):
        h, lc = self.h, self.lc
        slot = self.write_pos % 256
        self.ring_k[slot], self.ring_v[slot], self.ring_u[slot] = k_roped, v, k_unroped
        b_old = self.boundary
        self.boundary, self.write_pos, ev, c_len, win_len, win_start = KL.plan_step(
            self.boundary, self.write_pos, self.cap)
        if ev is not None:
            s0, r0, n = b_old % 256, b_old * H_KV, 128 * H_KV
            xk = np.ascontiguousarray(self.ring_u[s0:s0 + 128].reshape(n, D))
            xv = np.ascontiguousarray(self.ring_v[s0:s0 + 128].reshape(n, D))
            _, m, nk, rk, pk, sm = oracle.compress(xk, h["d_k"], h["rotor_k"], h["cents_k"],
                                                   h["cents_k"], ts=lc.ts_k, alpha=lc.alpha_k,
                                                   is_v=False)
            self.kmask[r0:r0 + n], self.knorm[r0:r0 + n], self.krn[r0:r0 + n] = m, nk, rk
            self.kpay[r0:r0 + n], self.vsm[r0:r0 + n] = pk, sm
            _, _, nv, rv, pv, sm = oracle.compress(xv, h["d_v"], h["rotor_v"], h["cents_v"],
                                                   h["vq"], ts=lc.ts_v, alpha=lc.alpha_v,
                                                   is_v=True)
            self.vnorm[r0:r0 + n], self.vrn[r0:r0 + n] = nv, rv
            self.vpay[r0:r0 + n], self.vsm[r0:r0 + n] = pv, sm
        has_c, has_w = c_len > 0, win_len > 0
        ac = aw = None
        if has_c:
            n_sp = KL.split_count(c_len, self.splits)
            _, ac, _ = oracle.attn(q_gate, self.kpay, self.vpay, self.vsm, self.kmask, self.knorm,
                                   self.krn, self.vnorm, self.vrn, h["cents_k"], h["cents_v"],
                                   h["vq"], h["rotor_k"], h["rotor_v"], h["d_k"], h["d_v"],
                                   num_queries=H_Q, num_heads=H_Q, L_q=1, c_len=c_len,
                                   n_rep=N_REP, scale=SCALE, alpha_k=lc.alpha_k,
                                   alpha_v=lc.alpha_v, rope_base=THETA, start_pos=0,
                                   num_splits=n_sp)
        if has_w:
            _, aw = oracle.window_attn(q_gate, self.ring_k, self.ring_v, win_start=win_start,
                                       win_len=win_len, ring_cap=256, H_q=H_Q, H_kv=H_KV,
                                       scale=SCALE)
        src_c = ac if has_c else aw
        _, out = oracle.merge_gate(src_c, aw, q_gate, H_q=H_Q, has_w=has_w and has_c)
        return out, ev


def _hip_d2d(dst: int, src: int, nbytes: int) -> int:
    """hipMemcpy device to device (kind 3) on raw pointers."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    return hip.hipMemcpy(dst, src, nbytes, 3)


def _tokens(n, seed):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n, H_KV, D)).astype(np.float16)
    v = rng.standard_normal((n, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((n, H_Q, 2 * D)).astype(np.float16)
    return k, rope_fp16_rows(k, np.arange(n)), v, q


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "reference-sequence"])
def test_layer_matches_simulation(device, fused):
    lc, h = layer_consts(layer_id=5)
    opt = KL.KhqOptions(splits=8, fused=fused, debug=True)
    L = KL.KhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    sim = Sim(lc, h, splits=8, cap=1024)
    k, kr, v, q = _tokens(N_STEPS, seed=3)
    out = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    checked = 0
    for t in range(N_STEPS):
        qt = torch.from_numpy(q[t]).to(device)
        ok = L.step(qt, torch.from_numpy(kr[t]).to(device), torch.from_numpy(v[t]).to(device),
                    out, SCALE, k_unroped=torch.from_numpy(k[t]).to(device))
        assert ok
        want, _ = sim.step(q[t], kr[t], v[t], k[t])
        if t % 13 == 0 or t in (255, 256, 383, 384, 511, 512, N_STEPS - 1):
            got = out.cpu().numpy().astype(np.float64)
            err = np.abs(got - want.astype(np.float64)).max()
            assert err <= 2e-3, (t, err)
            checked += 1
    assert checked > 40
    # cadence gate: event k at write_pos 256 + 128 (k-1), boundary 128 k, raw window 128
    assert [(e.write_pos, e.boundary, e.raw_window) for e in L.events] == \
        [(256, 128, 128), (384, 256, 128), (512, 384, 128)]
    # compressed rows identical to the oracle's (codes, norms, payloads)
    n = L.boundary * H_KV
    g = lambda x: x[:n].cpu().numpy()
    assert np.array_equal(g(L.pay.kmask).view(np.uint32), sim.kmask[:n])
    assert np.array_equal(g(L.pay.kpay), sim.kpay[:n])
    assert np.array_equal(g(L.pay.vpay), sim.vpay[:n])
    assert np.array_equal(g(L.pay.vsm), sim.vsm[:n])
    # norm fingerprint gate: each event's K norms match the true token norms,
    # and the true alignment beats +-128-token shifted alignments by 5x
    true_norm = np.linalg.norm(k.astype(np.float64), axis=2)  # [t, head]
    for e in L.events:
        b0 = e.boundary - 128
        bits = np.array(e.knorm_bits, np.uint16).view(np.float16).astype(np.float64)
        got = bits.reshape(128, H_KV)
        rel = np.mean(np.abs(got - true_norm[b0:b0 + 128]) / true_norm[b0:b0 + 128])
        assert rel <= 1e-2
        for shift in (-128, 128):
            lo = b0 + shift
            if 0 <= lo and lo + 128 <= N_STEPS:
                wrong = np.mean(np.abs(got - true_norm[lo:lo + 128]) / true_norm[lo:lo + 128])
                assert wrong > 5 * rel


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "reference-sequence"])
def test_native_layer_matches_python_layer(device, fused):
    """The C-ABI layer runtime (khq_layer_*) against the Python one: same
    kernels, so identical outputs, cadence and payload bytes, step by step."""
    lc, _ = layer_consts(layer_id=5)
    opt = KL.KhqOptions(splits=8, fused=fused)
    py = KL.KhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    na = KL.NativeKhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=1024, device=device, options=opt)
    k, kr, v, q = _tokens(400, seed=11)
    o1 = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    o2 = torch.empty_like(o1)
    for t in range(400):
        qt, kt, vt = (torch.from_numpy(a[t]).to(device) for a in (q, kr, v))
        ku = torch.from_numpy(k[t]).to(device)
        if t % 2:
            assert py.step(qt, kt, vt, o1, SCALE, k_unroped=ku)
            assert na.step(qt, kt, vt, o2, SCALE, k_unroped=ku)
        else:  # the reference's two-call order
            py.capture_unroped(ku)
            na.capture_unroped(ku)
            assert py.step(qt, kt, vt, o1, SCALE)
            assert na.step(qt, kt, vt, o2, SCALE)
        if t % 17 == 0 or t in (255, 256, 383, 384, 399):
            assert torch.equal(o1, o2), t
    assert na.state() == (py.boundary, py.write_pos, len(py.events)) == (256, 400, 2)
    ptrs = na.payload_ptrs()
    n = 256 * H_KV
    for i, name in enumerate(("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm")):
        ref = getattr(py.pay, name)[:n]
        got = torch.empty_like(ref)
        torch.cuda.synchronize()
        assert _hip_d2d(got.data_ptr(), ptrs[i], got.numel() * got.element_size()) == 0
        assert torch.equal(got, ref), name
    na.reset()
    assert na.state() == (0, 0, 0)


def test_capture_unroped_then_step(device):
    """The reference's two-call order: capture_unroped(k) before RoPE, then step."""
    lc, h = layer_consts(layer_id=6)
    L = KL.KhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=512, device=device,
                    options=KL.KhqOptions(splits=16))
    sim = Sim(lc, h, splits=16, cap=512)
    k, kr, v, q = _tokens(300, seed=4)
    out = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    for t in range(300):
        L.capture_unroped(torch.from_numpy(k[t]).to(device))
        L.step(torch.from_numpy(q[t]).to(device), torch.from_numpy(kr[t]).to(device),
               torch.from_numpy(v[t]).to(device), out, SCALE)
        want, _ = sim.step(q[t], kr[t], v[t], k[t])
    assert np.abs(out.cpu().numpy().astype(np.float64) - want).max() <= 2e-3
    assert L.boundary == 128 and L.write_pos == 300


def test_capacity_overflow_refused(device):
    lc, _ = layer_consts()
    L = KL.KhqLayer(lc, H_q=H_Q, H_kv=H_KV, cap=128, device=device)
    k, kr, v, q = _tokens(1, seed=5)
    qt, kt, vt = (torch.from_numpy(a[0]).to(device) for a in (q, kr, v))
    out = torch.empty((H_Q, D), device=device, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="exceeds"):
        for _ in range(400):
            L.step(qt, kt, vt, out, SCALE, k_unroped=torch.from_numpy(k[0]).to(device))
    assert L.boundary == 128


def test_runtime_loads_centroid_file(device, tmp_path):
    from khq import centroids as C

    path = tmp_path / "khq_calib.bin"
    C.write(str(path), [C.synthetic_layer(i) for i in (3, 7)])
    rt = KL.KhqRuntime(str(path), max_seq=512, device=device)
    L3 = rt.layer(3)
    assert rt.layer(3) is L3 and L3.cap == 512
    with pytest.raises(KeyError):
        rt.layer(4)
