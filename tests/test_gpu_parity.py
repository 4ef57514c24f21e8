"""GPU parity: libkhq_hip.so (through its C ABI) against the C oracle.

Bars: packed codes / masks / norms bit-exact; attention outputs within
max-abs 2e-3 and rel 1e-3 of the oracle's fp32 result (normalised acc, and the
logsumexp of each triple within 1e-3).
"""
import numpy as np
import pytest
import torch

import npref
import oracle
from khq import ops, synth
from khq.centroids import synthetic_layer
from khqdata import (D, H_KV, H_Q, N_REP, SCALE, THETA, layer_consts, oracle_attn,
                     oracle_window, random_rows_np, stressed_rows_np,
                     two_region_state)

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-3


@pytest.fixture(params=[0, 1], ids=["auto", "portable"])
def kernel(request, device):
    """Runs a test with each compressed-region kernel: automatic (wavefront-
    specialised matrix-core) and portable."""
    from khq import _lib

    _lib.call("khq_select_kernel", request.param)
    yield request.param
    _lib.call("khq_select_kernel", 0)


def t(a, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def close(got, want, atol=ATOL, rtol=RTOL):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    assert err.max() <= atol, f"max abs err {err.max():.3e}"
    rel = err.max() / max(np.abs(want).max(), 1e-30)
    assert rel <= rtol, f"rel err {rel:.3e}"


def margins(got, want):
    """(max-abs error / ATOL, relative error / RTOL) of the outputs: the share
    of each tolerance that the error uses (1 = at the bar)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    return err.max() / ATOL, err.max() / max(np.abs(want).max(), 1e-30) / RTOL


def check_triple(got, want):
    g, gl = npref.triple_to_out(got)
    w, wl = npref.triple_to_out(want)
    close(g, w)
    assert np.abs(gl - wl).max() <= 1e-3
    return margins(g, w)


def payload_from_rows(rows, n_rows, device="cuda"):
    pay = ops.Payload(n_rows, device)
    pay.kmask.copy_(t(rows["kmask"].view(np.int32)))
    for k in ("kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm"):
        getattr(pay, k).copy_(t(rows[k]))
    return pay


def cents_dev(lc, device="cuda"):
    return ops.Centroids(lc, device)


# ------------------------------------------------------------------ compress
@pytest.mark.parametrize("n", [1, 5, 512, 1001])
def test_compress_bitexact(device, n):
    lc, h = layer_consts()
    rng = np.random.default_rng(n)
    x = rng.standard_normal((n, D)).astype(np.float16)
    x[0] = 0  # zero row edge case
    if n > 4:  # rows with many outliers (cap 50 hit)
        x[1:3] *= np.float16(0)
        x[1, ::3] = 40.0
        x[2, :] = np.float16(1e-3)
        x[2, 7] = 30000.0
    cents = cents_dev(lc, device)
    pay = ops.Payload(n, device)
    xt = t(x)
    ops.compress(xt, cents, pay, 0, is_v=False)
    ops.compress(xt, cents, pay, 0, is_v=True)
    torch.cuda.synchronize()
    rc, kmask, knorm, krn, kpay, ksm = oracle.compress(x, h["d_k"], h["rotor_k"], h["cents_k"],
                                                       h["cents_k"], ts=lc.ts_k, alpha=lc.alpha_k,
                                                       is_v=False)
    rc, _, vnorm, vrn, vpay, vsm = oracle.compress(x, h["d_v"], h["rotor_v"], h["cents_v"],
                                                   h["vq"], ts=lc.ts_v, alpha=lc.alpha_v,
                                                   is_v=True)
    g = lambda a: a.cpu().numpy()
    assert np.array_equal(g(pay.kmask).view(np.uint32), kmask)
    assert np.array_equal(g(pay.kpay), kpay)
    assert np.array_equal(g(pay.knorm).view(np.uint16), knorm.view(np.uint16))
    assert np.array_equal(g(pay.krn).view(np.uint16), krn.view(np.uint16))
    assert np.array_equal(g(pay.vpay), vpay)
    assert np.array_equal(g(pay.vnorm).view(np.uint16), vnorm.view(np.uint16))
    assert np.array_equal(g(pay.vrn).view(np.uint16), vrn.view(np.uint16))
    assert np.array_equal(g(pay.vsm), vsm)  # V writes max residual after K wrote 0


def test_compress_bitexact_scaled_codebook(device):
    # alpha_v = 1/16 puts the codebook at the projection scale: real VQ decisions
    lc, h = layer_consts(alpha_v=1.0 / 16.0, ts_k=1.3)
    rng = np.random.default_rng(99)
    x = rng.standard_normal((256, D)).astype(np.float16)
    cents = cents_dev(lc, device)
    pay = ops.Payload(256, device)
    ops.compress(t(x), cents, pay, 0, is_v=False)
    ops.compress(t(x), cents, pay, 0, is_v=True)
    rc, kmask, _, krn, kpay, _ = oracle.compress(x, h["d_k"], h["rotor_k"], h["cents_k"],
                                                 h["cents_k"], ts=1.3, alpha=1.0, is_v=False)
    rc, _, _, vrn, vpay, vsm = oracle.compress(x, h["d_v"], h["rotor_v"], h["cents_v"], h["vq"],
                                               ts=1.95, alpha=1.0 / 16.0, is_v=True)
    assert np.array_equal(pay.kmask.cpu().numpy().view(np.uint32), kmask)
    assert np.array_equal(pay.kpay.cpu().numpy(), kpay)
    assert np.array_equal(pay.vpay.cpu().numpy(), vpay)
    assert np.array_equal(pay.vsm.cpu().numpy(), vsm)
    assert np.array_equal(pay.vrn.cpu().numpy().view(np.uint16), vrn.view(np.uint16))


def test_compress_error_codes(device):
    lib = __import__("khq._lib", fromlist=["lib"])
    rc = lib.call("launch_khq_compress_fp16", *([None] * 10), 0, 256, 1.0, 1.0, 0, None,
                  check=False)
    assert rc == -100
    rc = lib.call("launch_khq_compress_fp16", *([None] * 10), 4, 128, 1.0, 1.0, 0, None,
                  check=False)
    assert rc == -100


# ----------------------------------------------------------------- attention
def _gpu_state(st, device="cuda"):
    n_rows = st["rows"]["kmask"].shape[0]
    return payload_from_rows(st["rows"], n_rows, device), cents_dev(st["lc"], device)


def check_splits(got_part, want_part):
    """Split triples [q][split][258] of the reference partition: non-empty
    splits as triples, empty ones exactly (0, -1e20, 0) (ref .cu:1542-1553)."""
    got_part, want_part = np.asarray(got_part), np.asarray(want_part)
    assert got_part.shape == want_part.shape
    for sp in range(want_part.shape[1]):
        if want_part[0, sp, 257] == 0.0:
            assert np.all(got_part[:, sp, :256] == 0.0)
            assert np.all(got_part[:, sp, 256] == np.float32(-1e20))
            assert np.all(got_part[:, sp, 257] == 0.0)
        else:
            check_triple(got_part[:, sp], want_part[:, sp])


@pytest.mark.parametrize("splits", [1, 8])
def test_attn_c2(device, kernel, splits):
    st = two_region_state(seed=21)
    pay, cents = _gpu_state(st)
    out = torch.zeros((H_Q, D + 2), device=device)
    part = torch.full((H_Q, splits, D + 2), float("nan"), device=device)
    ops.attn(t(st["q_gate"]), pay, cents, out, c_len=st["c_len"], H_q=H_Q, H_kv=H_KV,
             scale=SCALE, num_splits=splits, out_partial=part if splits > 1 else None)
    torch.cuda.synchronize()
    rc, want, want_part = oracle_attn(st, num_splits=splits)
    check_triple(out.cpu().numpy(), want)
    if splits > 1:  # out_partial holds the reference's split triples
        check_splits(part.cpu().numpy(), want_part)


@pytest.mark.parametrize("c_len,splits", [(5, 8), (37, 3), (200, 7), (1000, 32), (4100, 64)])
def test_attn_split_partition(device, kernel, c_len, splits):
    """num_splits selects the reference's partition per = ceil(c_len / n_sp),
    with empty splits when c_len < n_sp; out_partial is written."""
    lc, h = layer_consts()
    rows = random_rows_np(c_len * H_KV, seed=100 + c_len)
    q = np.random.default_rng(c_len).standard_normal((H_Q, 2 * D)).astype(np.float16)
    st = dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len)
    pay = payload_from_rows(rows, c_len * H_KV, device)
    out = torch.zeros((H_Q, D + 2), device=device)
    part = torch.full((H_Q, splits, D + 2), float("nan"), device=device)
    ops.attn(t(q), pay, cents_dev(lc, device), out, c_len=c_len, H_q=H_Q, H_kv=H_KV,
             scale=SCALE, num_splits=splits, out_partial=part)
    torch.cuda.synchronize()
    rc, want, want_part = oracle_attn(st, num_splits=splits)
    check_triple(out.cpu().numpy(), want)
    check_splits(part.cpu().numpy(), want_part)


@pytest.mark.parametrize("c_len", [1, 7, 255, 256, 257, 1000])
def test_attn_random_rows(device, kernel, c_len):
    lc, h = layer_consts()
    rows = random_rows_np(c_len * H_KV, seed=c_len)
    q = np.random.default_rng(c_len).standard_normal((H_Q, 2 * D)).astype(np.float16)
    st = dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len)
    pay = payload_from_rows(rows, c_len * H_KV, device)
    out = torch.zeros((H_Q, D + 2), device=device)
    ops.attn(t(q), pay, cents_dev(lc, device), out, c_len=c_len, H_q=H_Q, H_kv=H_KV,
             scale=SCALE)
    torch.cuda.synchronize()
    m_abs, m_rel = check_triple(out.cpu().numpy(), oracle_attn(st)[1])
    print(f"c_len {c_len}: max-abs err / 2e-3 = {m_abs:.3f}, rel err / 1e-3 = {m_rel:.3f}",
          flush=True)
    assert m_abs <= 0.5 and m_rel <= 0.5, (m_abs, m_rel)


def test_attn_outliers_past_cap_and_mult_range(device, kernel):
    """Rows with more than 50 outliers and multipliers outside [0.1, 10]
    (khqdata.stressed_rows_np), over several tiles, both kernels."""
    c_len = 300
    lc, h = layer_consts()
    rows = stressed_rows_np(c_len * H_KV, seed=4242)
    q = np.random.default_rng(4243).standard_normal((H_Q, 2 * D)).astype(np.float16)
    st = dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len)
    pay = payload_from_rows(rows, c_len * H_KV, device)
    out = torch.zeros((H_Q, D + 2), device=device)
    ops.attn(t(q), pay, cents_dev(lc, device), out, c_len=c_len, H_q=H_Q, H_kv=H_KV,
             scale=SCALE)
    torch.cuda.synchronize()
    check_triple(out.cpu().numpy(), oracle_attn(st)[1])


def test_attn_lq_start_pos(device):
    st = two_region_state(seed=22)
    pay, cents = _gpu_state(st)
    out = torch.zeros((H_Q * 3, D + 2), device=device)
    ops.attn(t(st["q_gate"]), pay, cents, out, c_len=300, H_q=H_Q, H_kv=H_KV, scale=SCALE,
             L_q=3, start_pos=11)
    torch.cuda.synchronize()
    rc, want, _ = oracle_attn(st, c_len=300, L_q=3, start_pos=11)
    check_triple(out.cpu().numpy(), want)


def test_attn_error_codes(device):
    st = two_region_state(seed=23)
    pay, cents = _gpu_state(st)
    out = torch.zeros((H_Q, D + 2), device=device)
    q = t(st["q_gate"])
    assert ops.attn(q, pay, cents, out, c_len=0, H_q=H_Q, H_kv=H_KV, scale=SCALE,
                    check=False) == -100
    assert ops.attn(q, pay, cents, out, c_len=10, H_q=H_Q, H_kv=H_KV, scale=SCALE, num_splits=4,
                    out_partial=None, check=False) == -101


def test_window_and_merge(device, kernel):
    st = two_region_state(seed=24)
    pay, cents = _gpu_state(st)
    q = t(st["q_gate"])
    ac = torch.zeros((H_Q, D + 2), device=device)
    aw = torch.zeros((H_Q, D + 2), device=device)
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    ops.attn(q, pay, cents, ac, c_len=st["c_len"], H_q=H_Q, H_kv=H_KV, scale=SCALE)
    ops.window_attn(q, t(st["ring_k"]), t(st["ring_v"]), aw, win_start=st["win_start"],
                    win_len=st["win_len"], ring_cap=256, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    ops.merge_gate(ac, aw, q, out, H_q=H_Q, has_w=True)
    torch.cuda.synchronize()
    rc, wc, _ = oracle_attn(st)
    rc, ww = oracle_window(st)
    check_triple(aw.cpu().numpy(), ww)
    rc, want = oracle.merge_gate(wc, ww, st["q_gate"], H_q=H_Q, has_w=True)
    close(out.cpu().numpy(), want)
    # merge kernel alone on the oracle's triples (isolates the merge)
    out2 = torch.zeros_like(out)
    ops.merge_gate(t(wc), t(ww), q, out2, H_q=H_Q, has_w=True)
    torch.cuda.synchronize()
    close(out2.cpu().numpy(), want, atol=1e-3)
    # fused two-region step
    out3 = torch.zeros_like(out)
    ops.attn_step(q, pay, cents, t(st["ring_k"]), t(st["ring_v"]), out3, H_q=H_Q, H_kv=H_KV,
                  c_len=st["c_len"], win_start=st["win_start"], win_len=st["win_len"],
                  ring_cap=256, scale=SCALE)
    torch.cuda.synchronize()
    close(out3.cpu().numpy(), want)


@pytest.mark.parametrize("case", ["window-only", "compressed-only", "wrap-216", "full-ring"])
def test_fused_step_regions(device, kernel, case):
    """khq_attn_step_fp16 for each region combination the layer runtime issues,
    against the oracle's window / compressed triples merged and gated."""
    st = two_region_state(seed=31, n_tokens=600, boundary=384)
    c_len, win_start, win_len = 384, 384 % 256, 216
    if case == "window-only":
        c_len, win_start, win_len = 0, 0, 200
    elif case == "compressed-only":
        win_len = 0
    elif case == "full-ring":
        win_start, win_len = (600 - 256) % 256, 256
    st.update(c_len=c_len, win_start=win_start, win_len=win_len)
    pay, cents = _gpu_state(st)
    q = t(st["q_gate"])
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    ops.attn_step(q, pay, cents, t(st["ring_k"]), t(st["ring_v"]), out, H_q=H_Q, H_kv=H_KV,
                  c_len=c_len, win_start=win_start, win_len=win_len, ring_cap=256, scale=SCALE)
    torch.cuda.synchronize()
    if c_len == 0:
        _, ww = oracle_window(st)
        _, want = oracle.merge_gate(ww, ww, st["q_gate"], H_q=H_Q, has_w=False)
    elif win_len == 0:
        _, wc, _ = oracle_attn(st)
        _, want = oracle.merge_gate(wc, wc, st["q_gate"], H_q=H_Q, has_w=False)
    else:
        _, wc, _ = oracle_attn(st)
        _, ww = oracle_window(st)
        _, want = oracle.merge_gate(wc, ww, st["q_gate"], H_q=H_Q, has_w=True)
    close(out.cpu().numpy(), want)


def test_window_wrap_and_guards(device):
    st = two_region_state(seed=25, n_tokens=600, boundary=384)
    st["win_start"], st["win_len"] = 384 % 256, 216
    q = t(st["q_gate"])
    aw = torch.zeros((H_Q, D + 2), device=device)
    ops.window_attn(q, t(st["ring_k"]), t(st["ring_v"]), aw, win_start=128, win_len=216,
                    ring_cap=256, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    check_triple(aw.cpu().numpy(), oracle_window(st)[1])
    rk, rv = t(st["ring_k"]), t(st["ring_v"])
    assert ops.window_attn(q, rk, rv, aw, win_start=0, win_len=0, ring_cap=256, H_q=H_Q,
                           H_kv=H_KV, scale=SCALE, check=False) == -100
    assert ops.window_attn(q, rk, rv, aw, win_start=0, win_len=257, ring_cap=256, H_q=H_Q,
                           H_kv=H_KV, scale=SCALE, check=False) == -100


def test_gather_q_bitexact(device):
    q = np.random.default_rng(1).standard_normal((H_Q, 2 * D)).astype(np.float16)
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    ops.gather_q(t(q), out, H_q=H_Q)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), q[:, :D])


@pytest.mark.parametrize("win", [1, 17, 200, 256])
def test_c3_window_block_lengths(device, win):
    """At C3's size the fused step computes the raw window in one block of the
    decode launch (window_block_all: scores, softmax, P x V on the matrix
    cores with hi + lo weights).  Window lengths 1 (one half empty), 17, 200
    and 256 (the full ring) against the separate launches: compressed
    partials, window partials (window_part_kernel, oracle-checked) and the
    merge with gate."""
    lc, h = layer_consts(layer_id=2)
    c_len = 32640
    rows = random_rows_np(c_len * H_KV, seed=5)
    rng = np.random.default_rng(6 + win)
    q = rng.standard_normal((H_Q, 2 * D)).astype(np.float16)
    ring_k = t(rng.standard_normal((256, H_KV, D)).astype(np.float16))
    ring_v = t(rng.standard_normal((256, H_KV, D)).astype(np.float16))
    pay = payload_from_rows(rows, c_len * H_KV, device)
    cents = cents_dev(lc, device)
    ws = c_len % 256
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    ops.attn_step(t(q), pay, cents, ring_k, ring_v, out, H_q=H_Q, H_kv=H_KV, c_len=c_len,
                  win_start=ws, win_len=win, ring_cap=256, scale=SCALE)
    ac = torch.zeros((H_Q, D + 2), device=device)
    aw = torch.zeros((H_Q, D + 2), device=device)
    want = torch.zeros_like(out)
    ops.attn(t(q), pay, cents, ac, c_len=c_len, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    ops.window_attn(t(q), ring_k, ring_v, aw, win_start=ws, win_len=win, ring_cap=256, H_q=H_Q,
                    H_kv=H_KV, scale=SCALE)
    ops.merge_gate(ac, aw, t(q), want, H_q=H_Q, has_w=True)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), want.cpu().numpy())


@pytest.mark.parametrize("c_len", [4064, 8128, 12160, 20320])
def test_mid_context_chunking(device, c_len):
    """Contexts whose one-CU-spare split would use 253..255 chunks: with chunks
    of up to four tiles the split drops to at most n_cu - 4 chunks so the four
    per-KV-head window blocks run beside them (4064, 8128, 12160 tokens); with
    longer chunks (20320) it keeps n_cu - 1 chunks and the all-heads window
    block.  The fused step against the separate launches."""
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = (c_len + 15) // 16
    parts = ops.attn_parts(c_len)
    per = -(-tiles // parts)
    assert -(-tiles // per) == parts
    if per <= 4:
        assert parts + 4 <= n_cu, (c_len, parts)
    else:
        assert parts <= n_cu - 1
    lc, h = layer_consts(layer_id=3)
    rows = random_rows_np(c_len * H_KV, seed=c_len)
    rng = np.random.default_rng(c_len + 1)
    q = rng.standard_normal((H_Q, 2 * D)).astype(np.float16)
    ring_k = t(rng.standard_normal((256, H_KV, D)).astype(np.float16))
    ring_v = t(rng.standard_normal((256, H_KV, D)).astype(np.float16))
    pay = payload_from_rows(rows, c_len * H_KV, device)
    cents = cents_dev(lc, device)
    ws = c_len % 256
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)
    ops.attn_step(t(q), pay, cents, ring_k, ring_v, out, H_q=H_Q, H_kv=H_KV, c_len=c_len,
                  win_start=ws, win_len=128, ring_cap=256, scale=SCALE)
    ac = torch.zeros((H_Q, D + 2), device=device)
    aw = torch.zeros((H_Q, D + 2), device=device)
    want = torch.zeros_like(out)
    ops.attn(t(q), pay, cents, ac, c_len=c_len, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    ops.window_attn(t(q), ring_k, ring_v, aw, win_start=ws, win_len=128, ring_cap=256, H_q=H_Q,
                    H_kv=H_KV, scale=SCALE)
    ops.merge_gate(ac, aw, t(q), want, H_q=H_Q, has_w=True)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), want.cpu().numpy())
    # the compressed partials alone against the oracle at the smallest size
    if c_len == 4064:
        st = dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len)
        check_triple(ac.cpu().numpy(), oracle_attn(st)[1])


def test_c3_full_size(device, kernel):
    """Config 3 at its real shape: 32,640 compressed + 128 raw, vs the oracle."""
    lc, h = layer_consts(layer_id=0)
    c_len, win = 32640, 128
    rows = random_rows_np(c_len * H_KV, seed=3)
    q = np.random.default_rng(4).standard_normal((H_Q, 2 * D)).astype(np.float16)
    st = dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len)
    pay = payload_from_rows(rows, c_len * H_KV, device)
    cents = cents_dev(lc, device)
    out = torch.zeros((H_Q, D + 2), device=device)
    ops.attn(t(q), pay, cents, out, c_len=c_len, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    rc, want, _ = oracle_attn(st, num_splits=32)
    check_triple(out.cpu().numpy(), want)
    # num_splits = 64: the reference's 64 split triples in out_partial, and
    # their merge in out_attn
    out8 = torch.zeros_like(out)
    part = torch.full((H_Q, 64, D + 2), float("nan"), device=device)
    ops.attn(t(q), pay, cents, out8, c_len=c_len, H_q=H_Q, H_kv=H_KV, scale=SCALE,
             num_splits=64, out_partial=part)
    torch.cuda.synchronize()
    rc, want64, want_part = oracle_attn(st, num_splits=64)
    check_triple(out8.cpu().numpy(), want64)
    check_splits(part.cpu().numpy(), want_part)
    # determinism: same inputs, identical bits
    out_b = torch.zeros_like(out)
    ops.attn(t(q), pay, cents, out_b, c_len=c_len, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    assert torch.equal(out, out_b)


@pytest.mark.parametrize("data", ["uniform", "compressed"])
def test_c3_precision_margin(device, data):
    """How much of the output tolerance the C3 result uses, on both data sets
    (seeded uniform-random codes; the library's compression of N(0,1) K / V
    rows).  The key-side operands are rounded to fp16 (the fold and the roped
    key), so the margin is asserted with room to spare: errors at most half of
    max-abs 2e-3 and of rel 1e-3."""
    lc, h = layer_consts(layer_id=1)
    c_len = 32640
    cents = cents_dev(lc, device)
    if data == "uniform":
        rows = random_rows_np(c_len * H_KV, seed=31)
        pay = payload_from_rows(rows, c_len * H_KV, device)
    else:
        pay = ops.Payload(c_len * H_KV, device)
        synth.compressed_rows(pay, cents, seed=32)
        torch.cuda.synchronize()
        rows = {k: getattr(pay, k).cpu().numpy() for k in
                ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm")}
        rows["kmask"] = rows["kmask"].view(np.uint32)
    q = np.random.default_rng(33).standard_normal((H_Q, 2 * D)).astype(np.float16)
    st = dict(rows=rows, h=h, lc=lc, q_gate=q, c_len=c_len)
    out = torch.zeros((H_Q, D + 2), device=device)
    ops.attn(t(q), pay, cents, out, c_len=c_len, H_q=H_Q, H_kv=H_KV, scale=SCALE)
    torch.cuda.synchronize()
    _, want, _ = oracle_attn(st, num_splits=32)
    m_abs, m_rel = check_triple(out.cpu().numpy(), want)
    print(f"C3 {data}: max-abs err / 2e-3 = {m_abs:.3f}, rel err / 1e-3 = {m_rel:.3f}", flush=True)
    assert m_abs <= 0.5 and m_rel <= 0.5, (m_abs, m_rel)


def test_gqa_baseline_reference_cases(device):
    from test_oracle_pins import _modular_inputs, gqa_fp64

    # 512 positions: 64 parts of 8 (two slots per wavefront); 3000 and 5000:
    # 256 parts of 12 and 20 (a wavefront's slots in one part-filled group,
    # and in a full group of four plus one)
    for H_q, H_kv, seq, max_seq in [(24, 4, 8, 16), (4, 2, 16, 16), (4, 2, 1, 16), (24, 4, 512, 512),
                                    (24, 4, 3000, 3000), (24, 4, 5000, 5000)]:
        qg, k, v = _modular_inputs(H_q, H_kv, 256, max_seq)
        qg16, k16, v16 = (a.astype(np.float16) for a in (qg, k, v))
        out = torch.zeros((H_q, D), device=device, dtype=torch.float16)
        ops.gqa_attn(t(qg16.reshape(H_q, 512)), t(k16.reshape(max_seq, H_kv, D)),
                     t(v16.reshape(max_seq, H_kv, D)), out, seq_len=seq, H_q=H_q, H_kv=H_kv,
                     scale=1.0 / 16.0)
        torch.cuda.synchronize()
        want = gqa_fp64(qg16.astype(np.float64), k16.astype(np.float64),
                        v16.astype(np.float64), seq, H_q, H_kv, 256, 1.0 / 16.0)
        got = out.cpu().numpy().astype(np.float64).ravel()
        assert np.abs(got - want).max() / np.abs(want).max() <= 2e-3
    # the guard of ref tests/test_gqa_attention_gpu.mojo:183-208: head_dim != 256 refused
    assert ops.gqa_attn(t(qg16.reshape(H_q, 512)), t(k16.reshape(max_seq, H_kv, D)),
                        t(v16.reshape(max_seq, H_kv, D)), out, seq_len=4, H_q=4, H_kv=2,
                        head_dim=128, scale=0.1, check=False) == -100


def test_partial_rope_matches_oracle(device):
    H = 24
    j = np.arange(H * 512)
    x = (((j * 7919 + 1013) % 2000).astype(np.float32) * 0.002 - 2.0).astype(np.float16)
    for pos in (0, 511, 8191):
        xt = t(x.reshape(H, 512).copy())
        ops.partial_rope(xt, num_heads=H, pos=pos, stride=512)
        torch.cuda.synchronize()
        want = oracle.partial_rope_fp16(x.reshape(H, 512), num_heads=H, head_dim=256,
                                        rotary_dim=64, pos=pos, theta=1e7, stride=512)
        got = xt.cpu().numpy()
        assert np.abs(got.astype(np.float32) - want.astype(np.float32)).max() <= 2e-3
        assert np.array_equal(got[:, 64:], want[:, 64:])


def test_attn_reduce_entry(device):
    """khq_attn_reduce_f32 merges split triples like the oracle's reduce."""
    st = two_region_state(seed=25)
    rc, want, want_part = oracle_attn(st, num_splits=8)
    out = torch.zeros((H_Q, D + 2), device=device)
    ops.attn_reduce(t(want_part.astype(np.float32)), out, num_queries=H_Q, num_splits=8)
    torch.cuda.synchronize()
    check_triple(out.cpu().numpy(), want)


def test_handoff_timeout_is_reported(device):
    """A hand-off wait that gives up (forced from the host with a one-sleep
    bound; every kernel still exits normally) yields NaN output and sets the
    fault word; with the default bound the same step is correct again."""
    lc, h = layer_consts(layer_id=0)
    c_len, win = 32640, 128
    rows = random_rows_np(c_len * H_KV, seed=3)
    q = np.random.default_rng(4).standard_normal((H_Q, 2 * D)).astype(np.float16)
    pay = payload_from_rows(rows, c_len * H_KV, device)
    cents = cents_dev(lc, device)
    ring = torch.zeros((256, H_KV, D), device=device, dtype=torch.float16)
    out = torch.zeros((H_Q, D), device=device, dtype=torch.float16)

    def step():
        ops.attn_step(t(q), pay, cents, ring, ring, out, H_q=H_Q, H_kv=H_KV, c_len=c_len,
                      win_start=0, win_len=win, ring_cap=256, scale=SCALE)
        torch.cuda.synchronize()

    assert ops.fault_status(clear=True) == 0
    ops.set_spin_limit(1)
    try:
        step()
    finally:
        ops.set_spin_limit(0)
    flag = ops.fault_status(clear=True)
    print(f"fault word after a one-sleep bound: {flag}", flush=True)
    if flag:
        assert torch.isnan(out.float()).any()
    step()
    assert ops.fault_status(clear=True) == 0
    assert not torch.isnan(out.float()).any()
