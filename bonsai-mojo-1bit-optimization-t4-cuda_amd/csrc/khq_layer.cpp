// khq_layer.cpp -- per-layer KHQ runtime behind the C ABI (khq_layer_*).
//
// Native counterpart of the reference's per-layer state and step
// (ref:src/khq/runtime.mojo:77-152 KhqLayer, :395-429 khq_init_layer,
// :432-451 khq_capture_unroped, :454-613 khq_step): a 256-slot fp16 ring for
// roped K, V and unroped K, the packed payload for cap tokens, the boundary /
// write_pos cadence (compress 128 tokens once the raw window reaches 256) and
// the two-region attention, all issued on the caller's stream.  Per-layer
// constant tensors (centroids, rotors, d vectors) are device buffers owned by
// the caller; the layer owns its rings, payload and scratch.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <algorithm>
#include <new>

#include "khq.h"
#include "khq_internal.h"

namespace {

constexpr int kRing = 256;       // ref runtime.mojo:36
constexpr int kWatermark = 256;  // :37
constexpr int kChunk = 128;      // :38
constexpr int kMaxSplits = 64;   // workspace bound of the reference-sequence path
constexpr int kD = 256;

}  // namespace

struct khq_layer {
    int H_q = 0, H_kv = 0, cap = 0, splits = 1, fused = 1;
    float ts_k = 0, alpha_k = 0, ts_v = 0, alpha_v = 0, rope_base = 0;
    const void *cents_k = nullptr, *cents_v = nullptr, *vq = nullptr;
    const void *rotor_k = nullptr, *rotor_v = nullptr, *d_k = nullptr, *d_v = nullptr;
    // owned device memory
    __half *ring_k = nullptr, *ring_v = nullptr, *ring_u = nullptr;
    uint32_t* kmask = nullptr;
    uint8_t *kpay = nullptr, *vpay = nullptr, *vsm = nullptr;
    __half *knorm = nullptr, *krn = nullptr, *vnorm = nullptr, *vrn = nullptr;
    float *ac = nullptr, *aw = nullptr, *ap = nullptr;
    int boundary = 0, write_pos = 0, n_events = 0;
    // chunked prefill: dense fp16 keys [key][H_kv][256] and V^T [H_kv][256][ld]
    // (key = token position), compressed tokens [0, dec_hi) already decoded,
    // raw tokens [raw_lo, raw_hi) already copied (empty when raw_lo >= raw_hi)
    __half *dk = nullptr, *dvt = nullptr;
    int d_keys = 0, d_ld = 0, dec_hi = 0, raw_lo = 0, raw_hi = 0;
    // calibration dumps of khq_layer_attention_step (not owned)
    khq_dump* dump = nullptr;
    int dump_layer = 0;
};

namespace {

void release(khq_layer* L) {
    void* ptrs[] = {L->ring_k, L->ring_v, L->ring_u, L->kmask, L->kpay, L->vpay, L->vsm,
                    L->knorm, L->krn, L->vnorm, L->vrn, L->ac, L->aw, L->ap, L->dk, L->dvt};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
}

template <typename T>
bool alloc_zero(T** p, size_t bytes) {
    if (hipMalloc(reinterpret_cast<void**>(p), bytes) != hipSuccess) {
        *p = nullptr;
        return false;
    }
    return hipMemset(*p, 0, bytes) == hipSuccess;
}

// Compression event: ring slots [boundary % 256, + 128) -> payload rows of
// tokens [boundary, boundary + 128) (ref runtime.mojo:494-552).
void compress_jobs(const khq_layer* L, khq::CompressJob* kj, khq::CompressJob* vj) {
    const int kv = L->H_kv * kD;
    const int s0 = L->boundary % kRing;
    const size_t r0 = (size_t)L->boundary * L->H_kv;
    const int n = kChunk * L->H_kv;
    auto h = [](const void* p) { return static_cast<const __half*>(p); };
    *kj = khq::CompressJob{L->ring_u + (size_t)s0 * kv, h(L->d_k), h(L->rotor_k), h(L->cents_k),
                           h(L->cents_k), L->kmask + r0 * 16, L->knorm + r0, L->krn + r0,
                           L->kpay + r0 * 40, nullptr, n, L->ts_k, L->alpha_k};
    *vj = khq::CompressJob{L->ring_v + (size_t)s0 * kv, h(L->d_v), h(L->rotor_v), h(L->cents_v),
                           h(L->vq), L->kmask + r0 * 16, L->vnorm + r0, L->vrn + r0,
                           L->vpay + r0 * 104, L->vsm + r0 * 4, n, L->ts_v, L->alpha_v};
}

int compress_event(khq_layer* L, hipStream_t stream) {
    // K and V rows in one launch (the two jobs write disjoint outputs)
    khq::CompressJob kj, vj;
    compress_jobs(L, &kj, &vj);
    const hipError_t e = khq::launch_compress_pair(kj, vj, stream);
    if (e != hipSuccess) return (int)e;
    L->boundary += kChunk;
    L->n_events += 1;
    return 0;
}

bool event_due(const khq_layer* L, int write_pos) {  // ref runtime.mojo:494-497
    return write_pos - L->boundary >= kWatermark && L->boundary + kChunk <= L->cap;
}

// Decode of rows [d0, d0 + nd) into the dense key space at the same positions.
void decomp_args(const khq_layer* L, int d0, int nd, khq::DecompArgs* a) {
    a->kpay = L->kpay;
    a->vpay = L->vpay;
    a->vsm = L->vsm;
    a->kmask = L->kmask;
    a->knorm = L->knorm;
    a->krn = L->krn;
    a->vnorm = L->vnorm;
    a->vrn = L->vrn;
    a->cents_k = static_cast<const __half*>(L->cents_k);
    a->cents_v = static_cast<const __half*>(L->cents_v);
    a->vq = static_cast<const __half*>(L->vq);
    a->rotor_k = static_cast<const __half*>(L->rotor_k);
    a->rotor_v = static_cast<const __half*>(L->rotor_v);
    a->dk = static_cast<const __half*>(L->d_k);
    a->dv = static_cast<const __half*>(L->d_v);
    a->out_k = L->dk;
    a->out_vt = L->dvt;
    a->h_kv = L->H_kv;
    a->tok0 = d0;
    a->n_tok = nd;
    a->start_pos = 0;
    a->key0 = d0;
    a->ld_vt = L->d_ld;
    a->a_k = L->alpha_k;
    a->a_v = L->alpha_v;
    a->rope_base = L->rope_base;
}

// Compression event whose rows are also decoded into the dense key space
// (which holds every earlier row: dec_hi = boundary), with an optional
// independent gather (the chunk append) in the same launch.
int compress_event_decoded(khq_layer* L, const khq::GatherArgs* g, hipStream_t stream) {
    const int c_a = L->boundary;
    khq::CompressJob kj, vj;
    compress_jobs(L, &kj, &vj);
    khq::DecompArgs da{};
    decomp_args(L, c_a, kChunk, &da);
    const hipError_t e = khq::launch_compress_decode(kj, vj, da, g, stream);
    if (e != hipSuccess) return (int)e;
    L->boundary += kChunk;
    L->n_events += 1;
    L->dec_hi = c_a + kChunk;
    // V^T columns up to the decode's last 16-column block are rewritten
    L->raw_lo = std::max(L->raw_lo, c_a + (kChunk + 15) / 16 * 16);
    return 0;
}

int split_count(int c_len, int splits) {  // ref runtime.mojo:211-222
    if (splits <= 1 || c_len <= 0) return 1;
    return std::max(1, std::min(c_len / 8, splits));
}

}  // namespace

extern "C" {

khq_layer* khq_layer_create(int H_q, int H_kv, int cap_tokens, const void* centroids_k,
                            const void* centroids_v, const void* vq_centroids,
                            const void* k_rotor, const void* v_rotor, const void* d_vec_k,
                            const void* d_vec_v, float ts_k, float alpha_k, float ts_v,
                            float alpha_v, float rope_base, int splits, int fused) {
    if (H_kv <= 0 || H_q <= 0 || H_q % H_kv != 0 || H_q / H_kv > 8 || cap_tokens < kChunk ||
        !centroids_k || !centroids_v || !vq_centroids || !k_rotor || !v_rotor || !d_vec_k ||
        !d_vec_v)
        return nullptr;
    khq_layer* L = new (std::nothrow) khq_layer();
    if (!L) return nullptr;
    L->H_q = H_q;
    L->H_kv = H_kv;
    L->cap = cap_tokens;
    L->splits = std::max(1, std::min(splits, kMaxSplits));
    L->fused = fused ? 1 : 0;
    L->ts_k = ts_k;
    L->alpha_k = alpha_k;
    L->ts_v = ts_v;
    L->alpha_v = alpha_v;
    L->rope_base = rope_base;
    L->cents_k = centroids_k;
    L->cents_v = centroids_v;
    L->vq = vq_centroids;
    L->rotor_k = k_rotor;
    L->rotor_v = v_rotor;
    L->d_k = d_vec_k;
    L->d_v = d_vec_v;
    const size_t ring = (size_t)kRing * H_kv * kD * sizeof(__half);
    const size_t rows = (size_t)cap_tokens * H_kv;
    const size_t trip = (size_t)H_q * (kD + 2) * sizeof(float);
    const bool ok = alloc_zero(&L->ring_k, ring) && alloc_zero(&L->ring_v, ring) &&
                    alloc_zero(&L->ring_u, ring) && alloc_zero(&L->kmask, rows * 64) &&
                    alloc_zero(&L->kpay, rows * 40) && alloc_zero(&L->vpay, rows * 104) &&
                    alloc_zero(&L->vsm, rows * 4) && alloc_zero(&L->knorm, rows * 2) &&
                    alloc_zero(&L->krn, rows * 2) && alloc_zero(&L->vnorm, rows * 2) &&
                    alloc_zero(&L->vrn, rows * 2) && alloc_zero(&L->ac, trip) &&
                    alloc_zero(&L->aw, trip) && alloc_zero(&L->ap, trip * L->splits);
    if (!ok) {
        release(L);
        delete L;
        return nullptr;
    }
    return L;
}

void khq_layer_destroy(khq_layer* L) {
    if (!L) return;
    (void)hipDeviceSynchronize();
    release(L);
    delete L;
}

int khq_layer_reset(khq_layer* L) {
    if (!L) return -100;
    L->boundary = 0;
    L->write_pos = 0;
    L->n_events = 0;
    L->dec_hi = 0;
    L->raw_lo = L->raw_hi = 0;
    return 0;
}

int khq_layer_state(const khq_layer* L, int* boundary, int* write_pos, int* n_events) {
    if (!L) return -100;
    if (boundary) *boundary = L->boundary;
    if (write_pos) *write_pos = L->write_pos;
    if (n_events) *n_events = L->n_events;
    return 0;
}

int khq_layer_payload(const khq_layer* L, void** ptrs) {
    if (!L || !ptrs) return -100;
    void* p[] = {L->kmask, L->kpay, L->knorm, L->krn, L->vpay, L->vnorm, L->vrn, L->vsm,
                 L->ring_k, L->ring_v, L->ring_u};
    for (int i = 0; i < 11; i++) ptrs[i] = p[i];
    return 0;
}

int khq_layer_dense(const khq_layer* L, void** k, void** vt, int* ld_vt, int* n_decoded) {
    if (!L || !k || !vt || !ld_vt || !n_decoded) return -100;
    *k = L->dk;
    *vt = L->dvt;
    *ld_vt = L->d_ld;
    *n_decoded = L->dec_hi;
    return 0;
}

int khq_layer_capture_unroped(khq_layer* L, const void* k_unroped, hipStream_t stream) {
    if (!L || !k_unroped) return -100;
    const int slot = L->write_pos % kRing;
    return launch_khq_ring_write_fp16(nullptr, nullptr, L->ring_u, nullptr, nullptr, k_unroped,
                                      slot, L->H_kv * kD, stream);
}

// khq_step after the ring writes of the token (ref runtime.mojo:489-613).
static int step_after_ring_write(khq_layer* L, const void* q_gate, void* out, float scale,
                                 hipStream_t stream);

int khq_layer_step(khq_layer* L, const void* q_gate, const void* k_roped, const void* v,
                   const void* k_unroped, void* out, float scale, hipStream_t stream) {
    if (!L || !q_gate || !k_roped || !v || !out) return -100;
    const int kv = L->H_kv * kD;
    const int slot = L->write_pos % kRing;
    int rc = launch_khq_ring_write_fp16(L->ring_k, L->ring_v, k_unroped ? L->ring_u : nullptr,
                                        k_roped, v, k_unroped, slot, kv, stream);
    if (rc) return rc;
    return step_after_ring_write(L, q_gate, out, scale, stream);
}

int khq_layer_set_dump(khq_layer* L, khq_dump* dump, int layer_id) {
    if (!L || layer_id < 0) return -100;
    L->dump = dump;
    L->dump_layer = layer_id;
    return 0;
}

int khq_layer_attention_step(khq_layer* L, void* q_gate, void* k, const void* v,
                             const float* q_norm_w, const float* k_norm_w, float eps, int pos,
                             void* out, float scale, hipStream_t stream) {
    if (!L || !q_gate || !k || !v || !out || pos < 0 || !(eps >= 0.0f)) return -100;
    const int slot = L->write_pos % kRing;
    khq::NormRopeArgs a{};
    a.q_gate = static_cast<__half*>(q_gate);
    a.k = static_cast<__half*>(k);
    a.v = static_cast<const __half*>(v);
    a.q_w = q_norm_w;
    a.k_w = k_norm_w;
    a.ring_k = L->ring_k;
    a.ring_v = L->ring_v;
    a.ring_u = L->ring_u;
    a.H_q = L->H_q;
    a.H_kv = L->H_kv;
    a.slot = slot;
    a.pos = pos;
    a.rot = 64;  // the compressed kernels' rotary width (dims 0..63)
    a.eps = eps;
    a.theta = L->rope_base;
    hipError_t e = khq::launch_norm_rope(a, stream);
    if (e != hipSuccess) return (int)e;
    if (L->dump) {  // calibration dumps (ref attention.mojo:340-341, 355-356)
        const size_t kv = (size_t)L->H_kv * kD;
        int rc = khq_dump_kv(L->dump, L->dump_layer, L->ring_u + (size_t)slot * kv, v, stream);
        if (rc) return rc;
        rc = khq_dump_attn(L->dump, L->dump_layer, q_gate, k, pos, L->H_q, L->H_kv, kD, scale,
                           stream);
        if (rc) return rc;
    }
    return step_after_ring_write(L, q_gate, out, scale, stream);
}

static int step_after_ring_write(khq_layer* L, const void* q_gate, void* out, float scale,
                                 hipStream_t stream) {
    int rc = 0;
    L->raw_lo = L->raw_hi = 0;  // the dense key space does not get this token
    L->write_pos += 1;
    if (event_due(L, L->write_pos)) {
        rc = compress_event(L, stream);
        if (rc) return rc;
    }
    const int c_len = L->boundary;
    const int win_len = L->write_pos - c_len;
    if (c_len <= 0 && win_len <= 0) return 0;
    // The reference reads overwritten ring slots once cap is reached
    // (README:259); refuse instead.
    if (win_len > kRing) return -102;
    const int win_start = c_len % kRing;
    if (L->fused) {
        rc = khq_attn_step_fp16(q_gate, L->kpay, L->vpay, L->vsm, L->kmask, L->knorm, L->krn,
                                L->vnorm, L->vrn, L->cents_k, L->cents_v, L->vq, L->rotor_k,
                                L->rotor_v, L->d_k, L->d_v, L->ring_k, L->ring_v, out, L->H_q,
                                L->H_kv, c_len, win_start, win_len, kRing, scale, L->alpha_k,
                                L->alpha_v, L->rope_base, stream);
        return rc ? rc : 1;
    }
    const int has_c = c_len > 0, has_w = win_len > 0;
    if (has_c) {
        const int n_sp = split_count(c_len, L->splits);
        rc = launch_khq_attn_fp16(q_gate, L->kpay, L->vpay, L->vsm, L->kmask, L->knorm, L->krn,
                                  L->vnorm, L->vrn, L->cents_k, L->cents_v, L->vq, L->rotor_k,
                                  L->rotor_v, L->d_k, L->d_v, L->ac, n_sp > 1 ? L->ap : nullptr,
                                  L->H_q, L->H_q, 1, c_len, 0, L->H_q / L->H_kv, scale,
                                  L->alpha_k, L->alpha_v, L->rope_base, 0, n_sp, stream);
        if (rc) return rc;
    }
    if (has_w) {
        rc = launch_khq_window_attn_fp16(q_gate, L->ring_k, L->ring_v, L->aw, win_start, win_len,
                                         kRing, L->H_q, L->H_kv, kD, scale, stream);
        if (rc) return rc;
    }
    // has_c = 0: the window triple stands in for the compressed one
    // (ref ops.mojo:1255-1279)
    rc = launch_khq_merge_gate_fp16(has_c ? L->ac : L->aw, L->aw, q_gate, out, L->H_q, kD,
                                    has_c && has_w, stream);
    return rc ? rc : 1;
}

int khq_layer_prefill(khq_layer* L, const void* q_gate, const void* k_roped, const void* v,
                      const void* k_unroped, void* out, int n, float scale, hipStream_t stream) {
    if (!L || !q_gate || !k_roped || !v || !k_unroped || !out || n <= 0) return -100;
    const int kv = L->H_kv * kD;
    if (!L->dk) {  // dense key space for up to cap + 256 positions
        // positions up to cap + ring, then the raw copy of one compressed
        // chunk (the extra keys of a combined launch) past them
        L->d_keys = L->cap + kRing + kChunk + 64;
        L->d_ld = (L->d_keys + 63) / 64 * 64;
        const size_t kb = (size_t)L->d_keys * kv * sizeof(__half);
        const size_t vb = (size_t)L->H_kv * kD * L->d_ld * sizeof(__half);
        if (hipMalloc(reinterpret_cast<void**>(&L->dk), kb) != hipSuccess ||
            hipMalloc(reinterpret_cast<void**>(&L->dvt), vb) != hipSuccess) {
            if (L->dk) (void)hipFree(L->dk);
            L->dk = nullptr;
            L->dvt = nullptr;
            return -100;
        }
        // finite contents everywhere: padding keys of a launch get P = 0
        if (hipMemsetAsync(L->dk, 0, kb, stream) != hipSuccess ||
            hipMemsetAsync(L->dvt, 0, vb, stream) != hipSuccess) {
            // leave no half-initialised dense key space behind: the next
            // call allocates and clears it again
            (void)hipStreamSynchronize(stream);
            (void)hipFree(L->dk);
            (void)hipFree(L->dvt);
            L->dk = nullptr;
            L->dvt = nullptr;
            return -100;
        }
        L->dec_hi = 0;
    }
    const __half* qg = static_cast<const __half*>(q_gate);
    const __half* kr = static_cast<const __half*>(k_roped);
    const __half* vv = static_cast<const __half*>(v);
    const __half* ku = static_cast<const __half*>(k_unroped);
    __half* o = static_cast<__half*>(out);
    int done = 0;
    while (done < n) {
        // Sub-chunk whose ring writes overwrite no slot that any of its
        // queries or compression events still reads.
        const int m = std::min(n - done, kRing - (L->write_pos - L->boundary));
        if (m <= 0) return -102;
        const int w0 = L->write_pos;
        // An event due at the sub-chunk's last query and at none before it
        // (the usual case: the sub-chunk fills the ring to the watermark):
        // the event runs first and one attention launch serves every query;
        // the earlier queries read the chunk's raw rows from a copy past the
        // sub-chunk's keys instead of its decoded rows.
        const bool combine = m >= 2 && event_due(L, w0 + m) && !event_due(L, w0 + m - 1);
        const int c_a = L->boundary;
        const int side0 = (w0 + m + 15) / 16 * 16;
        // the sub-chunk's tokens go to their ring slots and to the dense key
        // space in one launch (with the raw copy as a second job)
        khq::GatherArgs cw{};
        cw.out_k = L->dk;
        cw.out_vt = L->dvt;
        cw.h_kv = L->H_kv;
        cw.win_start = w0 % kRing;
        cw.n = m;
        cw.ring_cap = kRing;
        cw.key0 = w0;
        cw.ld_vt = L->d_ld;
        cw.src_k = kr + (size_t)done * kv;
        cw.src_v = vv + (size_t)done * kv;
        cw.src_u = ku + (size_t)done * kv;
        cw.wr_k = L->ring_k;
        cw.wr_v = L->ring_v;
        cw.wr_u = L->ring_u;
        if (combine) {
            cw.side_n = kChunk;
            cw.side_start = c_a % kRing;
            cw.side_from_src = std::min(w0 - c_a, kChunk);
            cw.side_key0 = side0;
        }
        // With the compressed chunk wholly before the sub-chunk (the steady
        // state), the event reads no ring slot this launch writes: the append
        // then rides in the decode launch below instead of a launch of its own.
        const bool defer = combine && w0 >= c_a + kChunk && L->dec_hi < c_a + kChunk;
        if (!defer) {
            const hipError_t e = khq::launch_ring_gather(cw, stream);
            if (e != hipSuccess) return (int)e;
        }
        if (L->raw_lo < L->raw_hi && L->raw_hi == w0)
            L->raw_hi = w0 + m;
        else {
            L->raw_lo = w0;
            L->raw_hi = w0 + m;
        }
        // decoded rows up to c_len, raw rows [c_len, n_k) in the dense key space
        auto prepare = [&](int c_len, int n_k, const khq::GatherArgs* with) -> int {
            if (L->dec_hi < c_len) {
                const int d0 = L->dec_hi, nd = c_len - d0;
                int rc;
                if (with) {
                    khq::DecompArgs da{};
                    decomp_args(L, d0, nd, &da);
                    const hipError_t de = khq::launch_decompress_gather(da, *with, stream);
                    rc = de == hipSuccess ? 0 : (int)de;
                } else {
                    rc = khq_decompress_fp16(
                        L->kpay, L->vpay, L->vsm, L->kmask, L->knorm, L->krn, L->vnorm, L->vrn,
                        L->cents_k, L->cents_v, L->vq, L->rotor_k, L->rotor_v, L->d_k, L->d_v,
                        L->H_kv, d0, nd, 0, L->alpha_k, L->alpha_v, L->rope_base, L->dk, d0,
                        L->dvt, L->d_ld, stream);
                }
                if (rc) return rc;
                L->dec_hi = c_len;
                // V^T columns up to the decode's last 16-column block are rewritten
                L->raw_lo = std::max(L->raw_lo, d0 + (nd + 15) / 16 * 16);
            }
            // raw tokens [c_len, n_k): copied from the ring unless already
            // there (with every raw token after them, so the copy's padded
            // last block clobbers nothing still needed)
            if (!(L->raw_lo <= c_len && L->raw_hi >= n_k && L->raw_lo < L->raw_hi)) {
                const int g_hi = std::max(n_k, L->raw_lo < L->raw_hi && L->raw_lo <= n_k ? L->raw_hi : n_k);
                khq::GatherArgs g{};
                g.ring_k = L->ring_k;
                g.ring_v = L->ring_v;
                g.out_k = L->dk;
                g.out_vt = L->dvt;
                g.h_kv = L->H_kv;
                g.win_start = c_len % kRing;
                g.n = g_hi - c_len;
                g.ring_cap = kRing;
                g.key0 = c_len;
                g.ld_vt = L->d_ld;
                const hipError_t ge = khq::launch_ring_gather(g, stream);
                if (ge != hipSuccess) return (int)ge;
                L->raw_lo = c_len;
                L->raw_hi = g_hi;
            }
            return 0;
        };
        if (combine) {
            // steady state (every earlier row decoded): the event decodes its
            // own rows, with the deferred append in the same launch
            const bool fused = L->dec_hi == c_a;
            int rc = fused ? compress_event_decoded(L, defer ? &cw : nullptr, stream)
                           : compress_event(L, stream);
            if (rc) return rc;
            const int c_b = L->boundary;  // c_a + kChunk
            const int n_k = w0 + m;
            rc = prepare(c_b, n_k, defer && !fused ? &cw : nullptr);
            if (rc) return rc;
            rc = khq::prefill_attn_run(qg + (size_t)done * L->H_q * 2 * kD, L->dk, L->dvt,
                                       L->d_ld, n_k, m, w0 + 1, L->H_q, L->H_kv, scale,
                                       o + (size_t)done * L->H_q * kD, stream, m - 1, c_a, c_b,
                                       side0, side0 + (c_b - c_a));
            if (rc) return rc;
        }
        int j = combine ? m : 0;
        while (j < m) {
            // query j appends position w0 + j; an event fires before its attention
            if (event_due(L, w0 + j + 1)) {
                const int rc = compress_event(L, stream);
                if (rc) return rc;
            }
            int je = j + 1;
            while (je < m && !event_due(L, w0 + je + 1)) je++;
            // queries j .. je - 1 share c_len = boundary
            const int c_len = L->boundary;
            const int n_k = w0 + je;
            if (n_k - c_len > kRing) return -102;
            int rc = prepare(c_len, n_k, nullptr);
            if (rc) return rc;
            rc = khq_prefill_attn_fp16(qg + (size_t)(done + j) * L->H_q * 2 * kD, L->dk, L->dvt,
                                       L->d_ld, n_k, je - j, w0 + j + 1, L->H_q, L->H_kv, scale,
                                       o + (size_t)(done + j) * L->H_q * kD, stream);
            if (rc) return rc;
            j = je;
        }
        L->write_pos = w0 + m;
        done += m;
    }
    return n;
}

}  // extern "C"
