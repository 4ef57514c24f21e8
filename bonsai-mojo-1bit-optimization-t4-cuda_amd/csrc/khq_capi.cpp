// khq_capi.cpp -- extern "C" boundary of libkhq_hip.so (declared in
// include/khq.h).  Argument checks and return codes follow the reference
// launchers of ref:src/csrc/qmv_sm75_kernel.cu:4277-4429; the work split into
// kernels is this library's own.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "khq.h"
#include "khq_internal.h"

namespace {

constexpr int kMaxDevices = 64;

int rc_of(hipError_t e) { return e == hipSuccess ? 0 : static_cast<int>(e); }

// Device workspace for split partials, one per device, grown on demand
// (never shrunk; growing waits for the device).  Launches on different
// streams are ordered on the GPU: when a launch comes on another stream than
// the previous user of the workspace, the library records an event on the
// previous stream (all its work so far, the last use included) and makes the
// new stream wait for it, so two streams never use the workspace at once.
// A stream under graph capture is not ordered this way (a graph runs when it
// is replayed, not when it is captured): replays of a captured graph and
// eager launches on other streams must not overlap.  A buffer that a captured
// launch has used is never freed: when a later eager call needs more space,
// that buffer is retired (kept until the process ends) and a larger one
// allocated, so an earlier graph keeps replaying into memory it owns.  A
// captured call that would need to grow the workspace fails instead
// (hipErrorStreamCaptureUnsupported): reserve before capture.
struct Workspace {
    void* p = nullptr;
    size_t bytes = 0;
    bool used = false;
    bool in_graph = false;       // a captured graph holds this buffer's address
    hipStream_t last = nullptr;  // stream of the previous use
    hipEvent_t ev = nullptr;     // handed from the previous stream to the next
    std::vector<void*> retired;  // buffers captured graphs may still replay into
};
std::mutex g_ws_mu;
Workspace g_ws[kMaxDevices];

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// stream = the stream the caller launches on; reserve calls pass use = false
hipError_t workspace(size_t bytes, hipStream_t stream, float** out, bool use = true) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[dev];
    const bool cap = use && capturing(stream);
    if (w.bytes < bytes) {
        // growing under capture would bake a pointer that is freed later, and
        // the synchronisation it needs is illegal there: reserve beforehand
        if (cap) return hipErrorStreamCaptureUnsupported;
        size_t want = std::max(bytes, (size_t)4 << 20);
        if (w.p) {
            if (w.in_graph) {
                // a graph captured earlier replays into the old buffer: keep
                // it alive for the life of the process
                w.retired.push_back(w.p);
                w.in_graph = false;
            } else {
                e = hipDeviceSynchronize();
                if (e != hipSuccess) return e;
                e = hipFree(w.p);
                if (e != hipSuccess) return e;
            }
            w.p = nullptr;
            w.bytes = 0;
        }
        e = hipMalloc(&w.p, want);
        if (e != hipSuccess) return e;
        w.bytes = want;
    }
    if (use) {
        if (w.used && w.last != stream && !capturing(stream) && !capturing(w.last)) {
            if (!w.ev) {
                e = hipEventCreateWithFlags(&w.ev, hipEventDisableTiming);
                if (e != hipSuccess) return e;
            }
            e = hipEventRecord(w.ev, w.last);
            if (e != hipSuccess) return e;
            e = hipStreamWaitEvent(stream, w.ev, 0);
            if (e != hipSuccess) return e;
        }
        w.used = true;
        w.last = stream;
        if (cap) w.in_graph = true;
    }
    *out = static_cast<float*>(w.p);
    return hipSuccess;
}

std::mutex g_dev_mu;
std::atomic<int> g_cu_count[kMaxDevices] = {};  // 0 until first queried
struct LdsSet {
    const void* fn;
    int dev, bytes;
};
std::vector<LdsSet> g_lds_set;

// Partials of khq_attn_step_noalloc_fp16: a fixed device array per GPU
// (8 MiB, enough for H_q 24 at any context: at most 255 chunk parts + 64
// window parts of 258 floats per query head), never allocated at run time.
// Each device holds its own copy at its own address, which is looked up once
// per device (with that device current) and kept; the array's name is a
// host-side stand-in and is never passed to a kernel or a copy.  Every call
// on a GPU shares that GPU's array: calls that overlap on one GPU race.
constexpr size_t kScratchBytes = (size_t)8 << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {nullptr};

hipError_t scratch_ptr(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

// 0 = automatic (wavefront-specialised matrix-core kernel for the 24/4/256
// shape), 1 = portable lane-per-patch kernel for every shape.
std::atomic<int> g_kernel_choice{0};

bool use_mfma(int n_rep, int h_kv, int L_q) {
    return g_kernel_choice.load(std::memory_order_relaxed) != 1 && n_rep == 6 && h_kv == 4 && L_q == 1;
}

// Launches the compressed-region partials of query heads into part
// (stride part_stride, first index part_offset); returns the part count used.
hipError_t launch_compressed(khq::AttnArgs a, int n_rep, int L_q, int* parts_used,
                             hipStream_t stream) {
    if (use_mfma(n_rep, a.h_kv, L_q)) {
        int n_chunks = 0;
        const int per = khq::attn_ws_tiles_per_chunk(a.c_len, &n_chunks);
        *parts_used = n_chunks;
        return khq::launch_attn_ws(a, per, n_chunks, stream);
    }
    *parts_used = a.n_parts;
    return khq::launch_attn_parts(a, n_rep, dim3(a.n_parts, a.h_kv, L_q), stream);
}

int compressed_parts(int c_len, int n_rep, int h_kv, int L_q) {
    if (c_len <= 0) return 0;
    if (use_mfma(n_rep, h_kv, L_q)) {
        int n_chunks = 0;
        khq::attn_ws_tiles_per_chunk(c_len, &n_chunks);
        return n_chunks;
    }
    return std::max(1, std::min(256, (c_len + 31) / 32));
}

int window_parts(int win_len) { return std::max(1, std::min(64, (win_len + 3) / 4)); }

khq::AttnArgs attn_args(const void* q, const void* k_payload, const void* v_payload,
                        const void* v_shared_meta, const void* k_mask, const void* k_norms,
                        const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                        const void* centroids_k, const void* centroids_v,
                        const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                        const void* d_vec_k, const void* d_vec_v) {
    khq::AttnArgs a{};
    a.q = static_cast<const __half*>(q);
    a.kpay = static_cast<const uint8_t*>(k_payload);
    a.vpay = static_cast<const uint8_t*>(v_payload);
    a.vsm = static_cast<const uint8_t*>(v_shared_meta);
    a.kmask = static_cast<const uint32_t*>(k_mask);
    a.knorm = static_cast<const __half*>(k_norms);
    a.krn = static_cast<const __half*>(k_r_norms);
    a.vnorm = static_cast<const __half*>(v_norms);
    a.vrn = static_cast<const __half*>(v_r_norms);
    a.cents_k = static_cast<const __half*>(centroids_k);
    a.cents_v = static_cast<const __half*>(centroids_v);
    a.vq = static_cast<const __half*>(vq_centroids);
    a.rotor_k = static_cast<const __half*>(k_rotor);
    a.rotor_v = static_cast<const __half*>(v_rotor);
    a.dk = static_cast<const __half*>(d_vec_k);
    a.dv = static_cast<const __half*>(d_vec_v);
    return a;
}

}  // namespace

extern "C" {

const char* khq_version(void) { return "khq-mi355x 0.1 (gfx950)"; }

int khq_attn_parts(int c_len) { return compressed_parts(c_len, 6, 4, 1); }

int khq_select_kernel(int which) {
    if (which < 0 || which > 1) return -100;
    g_kernel_choice.store(which, std::memory_order_relaxed);
    return 0;
}

int khq_fault_status(int* flags, int clear) {
    if (!flags) return -100;
    return rc_of(khq::fault_status(flags, clear));
}

int khq_set_spin_limit(int sleeps) {
    if (sleeps < 0) return -100;
    khq::g_spin_limit.store(sleeps > 0 ? sleeps : (1 << 20), std::memory_order_relaxed);
    return 0;
}

int khq_workspace_reserve(size_t bytes) {
    float* p = nullptr;
    return rc_of(workspace(bytes, nullptr, &p, false));
}

int launch_khq_compress_fp16(const void* x, const void* d_vec, const void* rotor,
                             const void* centroids, const void* vq_centroids, void* out_mask,
                             void* out_norms, void* out_r_norms, void* out_payload,
                             void* out_shared_meta, int n, int d, float threshold_scale,
                             float alpha, int is_v, hipStream_t stream) {
    if (n <= 0 || d != 256) return -100;
    return rc_of(khq::launch_compress(
        static_cast<const __half*>(x), static_cast<const __half*>(d_vec),
        static_cast<const __half*>(rotor), static_cast<const __half*>(centroids),
        static_cast<const __half*>(vq_centroids), static_cast<uint32_t*>(out_mask),
        static_cast<__half*>(out_norms), static_cast<__half*>(out_r_norms),
        static_cast<uint8_t*>(out_payload), static_cast<uint8_t*>(out_shared_meta), n,
        threshold_scale, alpha, is_v ? 1 : 0, stream));
}

int launch_khq_attn_fp16(const void* q, const void* k_payload, const void* v_payload,
                         const void* v_shared_meta, const void* k_mask, const void* k_norms,
                         const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                         const void* centroids_k, const void* centroids_v,
                         const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                         const void* d_vec_k, const void* d_vec_v, void* out_attn,
                         void* out_partial, int num_queries, int num_heads, int L_q, int c_len,
                         int stride_s, int n_rep, float scale, float alpha_k, float alpha_v,
                         float rope_base, int start_pos, int num_splits, hipStream_t stream) {
    (void)stride_s;
    if (num_queries <= 0 || c_len <= 0) return -100;
    if (num_splits < 1) num_splits = 1;
    if (num_splits > 1 && out_partial == nullptr) return -101;
    // Shapes this library's kernels are built for.
    if (n_rep < 1 || n_rep > 8 || num_heads % n_rep != 0 || L_q < 1 ||
        num_queries != num_heads * L_q)
        return -100;
    const int h_kv = num_heads / n_rep;
    khq::AttnArgs a = attn_args(q, k_payload, v_payload, v_shared_meta, k_mask, k_norms,
                                k_r_norms, v_norms, v_r_norms, centroids_k, centroids_v,
                                vq_centroids, k_rotor, v_rotor, d_vec_k, d_vec_v);
    a.c_len = c_len;
    a.h_kv = h_kv;
    a.L_q = L_q;
    a.start_pos = start_pos;
    a.part_offset = 0;
    a.sc = scale;
    a.a_k = alpha_k;
    a.a_v = alpha_v;
    a.rope_base = rope_base;
    float* outp = static_cast<float*>(out_partial);
    hipError_t e;
    if (num_splits > 1 && !use_mfma(n_rep, h_kv, L_q)) {
        // the portable kernel cuts the tokens exactly as the reference does
        // (per = ceil(s_limit / n_sp), .cu:1542-1553) and writes the split
        // triples straight into out_partial [query][split][258]
        a.part = outp;
        a.n_parts = num_splits;
        a.part_stride = num_splits;
        e = khq::launch_attn_parts(a, n_rep, dim3(num_splits, h_kv, L_q), stream);
        if (e != hipSuccess) return rc_of(e);
        return rc_of(khq::launch_lse_reduce(outp, static_cast<float*>(out_attn), num_queries,
                                            num_splits, stream));
    }
    if (num_splits > 1) {
        // Matrix-core kernel: each reference split [sp * per, (sp + 1) * per)
        // is cut into `subs` chunks of whole tiles, so no chunk straddles a
        // split; the chunk triples merge into out_partial (the reference's
        // split triples, empty splits (0, -1e20, 0)), and those into out_attn.
        const int per = (c_len + num_splits - 1) / num_splits;
        const int split_tiles = (per + 15) / 16;
        const int want = std::max(1, std::min(split_tiles, 255 / num_splits));
        const int tpc = (split_tiles + want - 1) / want;
        const int subs = (split_tiles + tpc - 1) / tpc;
        const int nch = num_splits * subs;
        float* part = outp;
        if (subs > 1) {
            float* ws = nullptr;
            e = workspace((size_t)num_queries * nch * 258 * sizeof(float), stream, &ws);
            if (e != hipSuccess) return rc_of(e);
            part = ws;
        }
        a.part = part;
        a.n_parts = nch;
        a.part_stride = nch;
        a.split_per = per;
        a.split_subs = subs;
        e = khq::launch_attn_ws(a, tpc, nch, stream);
        if (e != hipSuccess) return rc_of(e);
        if (subs > 1) {
            e = khq::launch_lse_reduce(part, outp, num_queries * num_splits, subs, stream);
            if (e != hipSuccess) return rc_of(e);
        }
        return rc_of(khq::launch_lse_reduce(outp, static_cast<float*>(out_attn), num_queries,
                                            num_splits, stream));
    }
    // num_splits = 1: the library's own partition in its workspace, merged
    // into out_attn (the reference computes the same triple in one pass)
    const int np = compressed_parts(L_q > 1 ? std::min(c_len, L_q) : c_len, n_rep, h_kv, L_q);
    float* ws = nullptr;
    e = workspace((size_t)num_queries * np * 258 * sizeof(float), stream, &ws);
    if (e != hipSuccess) return rc_of(e);
    a.part = ws;
    a.n_parts = np;
    a.part_stride = np;
    int used = 0;
    e = launch_compressed(a, n_rep, L_q, &used, stream);
    if (e != hipSuccess) return rc_of(e);
    return rc_of(khq::launch_lse_reduce(ws, static_cast<float*>(out_attn), num_queries, np,
                                        stream));
}

int khq_attn_reduce_f32(const void* partial, void* out_attn, int num_queries, int num_splits,
                        hipStream_t stream) {
    if (!partial || !out_attn || num_queries <= 0 || num_splits < 1) return -100;
    return rc_of(khq::launch_lse_reduce(static_cast<const float*>(partial),
                                        static_cast<float*>(out_attn), num_queries, num_splits,
                                        stream));
}

int launch_khq_window_attn_fp16(const void* q, const void* ring_k, const void* ring_v,
                                void* out_attn, int win_start, int win_len, int ring_cap, int H_q,
                                int H_kv, int d, float scale, hipStream_t stream) {
    if (H_q <= 0 || win_len <= 0) return -100;
    if (d != 256 || H_kv <= 0 || H_q % H_kv != 0 || H_q / H_kv > 8 || ring_cap <= 0 ||
        win_len > ring_cap || win_start < 0)
        return -100;
    const int np = window_parts(win_len);
    float* ws = nullptr;
    hipError_t e = workspace((size_t)H_q * np * 258 * sizeof(float), stream, &ws);
    if (e != hipSuccess) return rc_of(e);
    khq::WinArgs w{};
    w.q = static_cast<const __half*>(q);
    w.ring_k = static_cast<const __half*>(ring_k);
    w.ring_v = static_cast<const __half*>(ring_v);
    w.part = ws;
    w.win_start = win_start;
    w.win_len = win_len;
    w.ring_cap = ring_cap;
    w.h_kv = H_kv;
    w.n_parts = np;
    w.part_stride = np;
    w.part_offset = 0;
    w.sc = scale;
    e = khq::launch_window_parts(w, H_q / H_kv, dim3(np, H_kv), stream);
    if (e != hipSuccess) return rc_of(e);
    return rc_of(khq::launch_lse_reduce(ws, static_cast<float*>(out_attn), H_q, np, stream));
}

int launch_khq_gather_q_fp16(const void* q_gate, void* q_out, int H_q, int d,
                             hipStream_t stream) {
    if (H_q <= 0 || d <= 0) return -100;
    return rc_of(khq::launch_gather_q(static_cast<const __half*>(q_gate),
                                      static_cast<__half*>(q_out), H_q, d, stream));
}

int launch_khq_merge_gate_fp16(const void* attn_c, const void* attn_w, const void* q_gate,
                               void* out, int H_q, int d, int has_w, hipStream_t stream) {
    if (H_q <= 0 || d <= 0) return -100;
    return rc_of(khq::launch_merge_gate(static_cast<const float*>(attn_c),
                                        static_cast<const float*>(attn_w),
                                        static_cast<const __half*>(q_gate),
                                        static_cast<__half*>(out), H_q, d, has_w ? 1 : 0,
                                        stream));
}

int launch_khq_ring_write_fp16(void* ring_k, void* ring_v, void* ring_u, const void* k_roped,
                               const void* v, const void* k_unroped, int slot, int kv,
                               hipStream_t stream) {
    if (kv <= 0 || slot < 0) return -100;
    if ((ring_k == nullptr) != (k_roped == nullptr) || (ring_v == nullptr) != (v == nullptr) ||
        (ring_u == nullptr) != (k_unroped == nullptr))
        return -100;
    if (ring_k == nullptr && ring_v == nullptr && ring_u == nullptr) return -100;
    const size_t off = (size_t)slot * kv;
    __half* rk = ring_k ? static_cast<__half*>(ring_k) + off : nullptr;
    __half* rv = ring_v ? static_cast<__half*>(ring_v) + off : nullptr;
    __half* ru = ring_u ? static_cast<__half*>(ring_u) + off : nullptr;
    return rc_of(khq::launch_ring_write(rk, rv, ru,
                                        static_cast<const __half*>(k_roped),
                                        static_cast<const __half*>(v),
                                        static_cast<const __half*>(k_unroped), kv, stream));
}

int launch_khq_partial_rope_fp16(void* vec, int num_heads, int head_dim, int rotary_dim,
                                 int pos, float theta_base, int stride, hipStream_t stream) {
    if (num_heads <= 0 || head_dim <= 0 || rotary_dim <= 0 || rotary_dim > head_dim ||
        (rotary_dim & 1))
        return -100;
    return rc_of(khq::launch_partial_rope(static_cast<__half*>(vec), num_heads, head_dim,
                                          rotary_dim, pos, theta_base, stride, stream));
}

int launch_khq_gqa_attn_fp16(const void* q_gate, const void* k_cache, const void* v_cache,
                             void* out, int seq_len, int H_q, int H_kv, int head_dim,
                             float scale, hipStream_t stream) {
    // The reference launcher refuses head_dim != 256 (tests/test_gqa_attention_gpu.mojo:183-208).
    if (head_dim != 256 || seq_len <= 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 ||
        H_q / H_kv > 8)
        return -100;
    // 8 positions per part (two per wavefront): 512 positions fill 256 blocks
    const int np = std::max(1, std::min(256, (seq_len + 7) / 8));
    float* ws = nullptr;
    hipError_t e = workspace((size_t)H_q * np * 258 * sizeof(float), stream, &ws);
    if (e != hipSuccess) return rc_of(e);
    khq::WinArgs w{};
    w.q = static_cast<const __half*>(q_gate);
    w.ring_k = static_cast<const __half*>(k_cache);
    w.ring_v = static_cast<const __half*>(v_cache);
    w.part = ws;
    w.win_start = 0;
    w.win_len = seq_len;
    w.ring_cap = seq_len;
    w.h_kv = H_kv;
    w.n_parts = np;
    w.part_stride = np;
    w.part_offset = 0;
    w.sc = scale;
    e = khq::launch_window_parts(w, H_q / H_kv, dim3(np, H_kv), stream);
    if (e != hipSuccess) return rc_of(e);
    // merge of the parts with every load issued up front (the window is all parts)
    khq::FinishArgs f{};
    f.part = ws;
    f.n_parts = np;
    f.part_stride = np;
    f.q = static_cast<const __half*>(q_gate);
    f.h_kv = H_kv;
    f.n_rep = H_q / H_kv;
    f.sc = scale;
    f.eps = 1e-9f;
    f.out = static_cast<__half*>(out);
    return rc_of(khq::launch_step_finish(f, H_q, stream));
}

int khq_attn_partials_fp16(const void* q_gate, const void* k_payload, const void* v_payload,
                           const void* v_shared_meta, const void* k_mask, const void* k_norms,
                           const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                           const void* centroids_k, const void* centroids_v,
                           const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                           const void* d_vec_k, const void* d_vec_v, int H_q, int H_kv,
                           int c_len, float scale, float alpha_k, float alpha_v,
                           float rope_base, hipStream_t stream) {
    if (c_len <= 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || H_q / H_kv > 8) return -100;
    const int npc = compressed_parts(c_len, H_q / H_kv, H_kv, 1);
    float* ws = nullptr;
    hipError_t e = workspace((size_t)H_q * npc * 258 * sizeof(float), stream, &ws);
    if (e != hipSuccess) return rc_of(e);
    khq::AttnArgs a = attn_args(q_gate, k_payload, v_payload, v_shared_meta, k_mask, k_norms,
                                k_r_norms, v_norms, v_r_norms, centroids_k, centroids_v,
                                vq_centroids, k_rotor, v_rotor, d_vec_k, d_vec_v);
    a.part = ws;
    a.c_len = c_len;
    a.h_kv = H_kv;
    a.L_q = 1;
    a.start_pos = 0;
    a.n_parts = npc;
    a.part_stride = npc;
    a.part_offset = 0;
    a.sc = scale;
    a.a_k = alpha_k;
    a.a_v = alpha_v;
    a.rope_base = rope_base;
    int used = 0;
    return rc_of(launch_compressed(a, H_q / H_kv, 1, &used, stream));
}

}  // extern "C"

static int attn_step_impl(const void* q_gate, const void* k_payload, const void* v_payload,
                       const void* v_shared_meta, const void* k_mask, const void* k_norms,
                       const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                       const void* centroids_k, const void* centroids_v,
                       const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                       const void* d_vec_k, const void* d_vec_v, const void* ring_k,
                       const void* ring_v, void* out, int H_q, int H_kv, int c_len,
                       int win_start, int win_len, int ring_cap, float scale, float alpha_k,
                       float alpha_v, float rope_base, hipStream_t stream,
                          bool noalloc) {
    if (c_len < 0 || win_len < 0 || (c_len == 0 && win_len == 0)) return -100;
    if (H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || H_q / H_kv > 8) return -100;
    if (win_len > 0 && (ring_cap <= 0 || win_len > ring_cap || win_start < 0)) return -100;
    const int n_rep = H_q / H_kv;
    const int npc = compressed_parts(c_len, n_rep, H_kv, 1);
    // Short windows (the KHQ ring holds 256 slots): window, merge and gate
    // without window partials.  With the wavefront-specialised kernel the
    // window is one extra block of the compressed launch (partial npc) and the
    // finishing launch only merges; otherwise the finishing launch computes
    // the window too.  Longer windows: window partials + combine.
    const bool fused_tail = win_len <= 256 && npc <= 1000;
    const bool win_in_ws = fused_tail && npc > 0 && win_len > 0 &&
                           g_kernel_choice.load(std::memory_order_relaxed) == 0 &&
                           use_mfma(n_rep, H_kv, 1);
    const int npw = (win_len > 0 && !fused_tail) ? window_parts(win_len) : (win_in_ws ? 1 : 0);
    const int np = npc + npw;
    const size_t ws_bytes = (size_t)H_q * std::max(np, 1) * 258 * sizeof(float);
    float* ws = nullptr;
    hipError_t e;
    if (noalloc) {
        if (ws_bytes > kScratchBytes) return -103;
        e = scratch_ptr(&ws);
    } else {
        e = workspace(ws_bytes, stream, &ws);
    }
    if (e != hipSuccess) return rc_of(e);
    const int ring = ring_cap > 0 ? ring_cap : 1;
    if (npc > 0) {
        khq::AttnArgs a = attn_args(q_gate, k_payload, v_payload, v_shared_meta, k_mask,
                                    k_norms, k_r_norms, v_norms, v_r_norms, centroids_k,
                                    centroids_v, vq_centroids, k_rotor, v_rotor, d_vec_k,
                                    d_vec_v);
        a.part = ws;
        a.c_len = c_len;
        a.h_kv = H_kv;
        a.L_q = 1;
        a.start_pos = 0;
        a.n_parts = npc;
        a.part_stride = np;
        a.part_offset = 0;
        a.sc = scale;
        a.a_k = alpha_k;
        a.a_v = alpha_v;
        a.rope_base = rope_base;
        if (win_in_ws) {
            a.ring_k = static_cast<const __half*>(ring_k);
            a.ring_v = static_cast<const __half*>(ring_v);
            a.win_start = win_start % ring;
            a.win_len = win_len;
            a.ring_cap = ring;
        }
        int used = 0;
        e = launch_compressed(a, n_rep, 1, &used, stream);
        if (e != hipSuccess) return rc_of(e);
    }
    if (fused_tail) {
        khq::FinishArgs f{};
        f.part = ws;
        f.n_parts = np;
        f.part_stride = np;
        f.q = static_cast<const __half*>(q_gate);
        f.ring_k = static_cast<const __half*>(ring_k);
        f.ring_v = static_cast<const __half*>(ring_v);
        f.ring_cap = ring;
        f.win_start = win_start % ring;
        f.win_len = win_in_ws ? 0 : win_len;
        f.h_kv = H_kv;
        f.n_rep = n_rep;
        f.sc = scale;
        f.eps = 1e-8f;
        f.out = static_cast<__half*>(out);
        return rc_of(khq::launch_step_finish(f, H_q, stream));
    }
    if (npw > 0) {
        khq::WinArgs w{};
        w.q = static_cast<const __half*>(q_gate);
        w.ring_k = static_cast<const __half*>(ring_k);
        w.ring_v = static_cast<const __half*>(ring_v);
        w.part = ws;
        w.win_start = win_start;
        w.win_len = win_len;
        w.ring_cap = ring_cap;
        w.h_kv = H_kv;
        w.n_parts = npw;
        w.part_stride = np;
        w.part_offset = npc;
        w.sc = scale;
        e = khq::launch_window_parts(w, n_rep, dim3(npw, H_kv), stream);
        if (e != hipSuccess) return rc_of(e);
    }
    return rc_of(khq::launch_combine_gate(ws, static_cast<const __half*>(q_gate),
                                          static_cast<__half*>(out), H_q, np, 1e-8f, stream));
}

extern "C" {

int khq_attn_step_fp16(const void* q_gate, const void* k_payload, const void* v_payload,
                       const void* v_shared_meta, const void* k_mask, const void* k_norms,
                       const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                       const void* centroids_k, const void* centroids_v,
                       const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                       const void* d_vec_k, const void* d_vec_v, const void* ring_k,
                       const void* ring_v, void* out, int H_q, int H_kv, int c_len,
                       int win_start, int win_len, int ring_cap, float scale, float alpha_k,
                       float alpha_v, float rope_base, hipStream_t stream) {
    return attn_step_impl(q_gate, k_payload, v_payload, v_shared_meta, k_mask, k_norms,
                          k_r_norms, v_norms, v_r_norms, centroids_k, centroids_v,
                          vq_centroids, k_rotor, v_rotor, d_vec_k, d_vec_v, ring_k, ring_v,
                          out, H_q, H_kv, c_len, win_start, win_len, ring_cap, scale,
                          alpha_k, alpha_v, rope_base, stream, false);
}

int khq_attn_step_noalloc_fp16(const void* q_gate, const void* k_payload, const void* v_payload,
                       const void* v_shared_meta, const void* k_mask, const void* k_norms,
                       const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                       const void* centroids_k, const void* centroids_v,
                       const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                       const void* d_vec_k, const void* d_vec_v, const void* ring_k,
                       const void* ring_v, void* out, int H_q, int H_kv, int c_len,
                       int win_start, int win_len, int ring_cap, float scale, float alpha_k,
                       float alpha_v, float rope_base, hipStream_t stream) {
    return attn_step_impl(q_gate, k_payload, v_payload, v_shared_meta, k_mask, k_norms,
                          k_r_norms, v_norms, v_r_norms, centroids_k, centroids_v,
                          vq_centroids, k_rotor, v_rotor, d_vec_k, d_vec_v, ring_k, ring_v,
                          out, H_q, H_kv, c_len, win_start, win_len, ring_cap, scale,
                          alpha_k, alpha_v, rope_base, stream, true);
}

int khq_decompress_fp16(const void* k_payload, const void* v_payload, const void* v_shared_meta,
                        const void* k_mask, const void* k_norms, const void* k_r_norms,
                        const void* v_norms, const void* v_r_norms, const void* centroids_k,
                        const void* centroids_v, const void* vq_centroids, const void* k_rotor,
                        const void* v_rotor, const void* d_vec_k, const void* d_vec_v, int H_kv,
                        int tok0, int n_tok, int start_pos, float alpha_k, float alpha_v,
                        float rope_base, void* out_k, int key0, void* out_vt, int ld_vt,
                        hipStream_t stream) {
    if (H_kv <= 0 || tok0 < 0 || n_tok < 0 || key0 < 0 || key0 % 8 != 0 || !out_k || !out_vt)
        return -100;
    if (ld_vt % 8 != 0 || ld_vt < key0 + (n_tok + 63) / 64 * 64) return -100;
    khq::DecompArgs a{};
    a.kpay = static_cast<const uint8_t*>(k_payload);
    a.vpay = static_cast<const uint8_t*>(v_payload);
    a.vsm = static_cast<const uint8_t*>(v_shared_meta);
    a.kmask = static_cast<const uint32_t*>(k_mask);
    a.knorm = static_cast<const __half*>(k_norms);
    a.krn = static_cast<const __half*>(k_r_norms);
    a.vnorm = static_cast<const __half*>(v_norms);
    a.vrn = static_cast<const __half*>(v_r_norms);
    a.cents_k = static_cast<const __half*>(centroids_k);
    a.cents_v = static_cast<const __half*>(centroids_v);
    a.vq = static_cast<const __half*>(vq_centroids);
    a.rotor_k = static_cast<const __half*>(k_rotor);
    a.rotor_v = static_cast<const __half*>(v_rotor);
    a.dk = static_cast<const __half*>(d_vec_k);
    a.dv = static_cast<const __half*>(d_vec_v);
    a.out_k = static_cast<__half*>(out_k);
    a.out_vt = static_cast<__half*>(out_vt);
    a.h_kv = H_kv;
    a.tok0 = tok0;
    a.n_tok = n_tok;
    a.start_pos = start_pos;
    a.key0 = key0;
    a.ld_vt = ld_vt;
    a.a_k = alpha_k;
    a.a_v = alpha_v;
    a.rope_base = rope_base;
    return rc_of(khq::launch_decompress(a, stream));
}

int khq_prefill_attn_fp16(const void* q_gate, const void* k, const void* vt, int ld_vt, int n_k,
                          int n_q, int vis0, int H_q, int H_kv, float scale, void* out,
                          hipStream_t stream) {
    if (!q_gate || !k || !vt || !out) return -100;
    return khq::prefill_attn_run(static_cast<const __half*>(q_gate), static_cast<const __half*>(k),
                                 static_cast<const __half*>(vt), ld_vt, n_k, n_q, vis0, H_q, H_kv,
                                 scale, static_cast<__half*>(out), stream, 0, 0, 0, 0, 0, true);
}

int khq_prefill_attn_partials_fp16(const void* q_gate, const void* k, const void* vt, int ld_vt,
                                   int n_k, int n_q, int vis0, int H_q, int H_kv, float scale,
                                   hipStream_t stream) {
    if (!q_gate || !k || !vt) return -100;
    return khq::prefill_attn_run(static_cast<const __half*>(q_gate), static_cast<const __half*>(k),
                                 static_cast<const __half*>(vt), ld_vt, n_k, n_q, vis0, H_q, H_kv,
                                 scale, nullptr, stream, 0, 0, 0, 0, 0, false);
}

int khq_attn_step_batched_fp16(const khq_seq* seqs, int n_seq, const void* centroids_k,
                               const void* centroids_v, const void* vq_centroids,
                               const void* k_rotor, const void* v_rotor, const void* d_vec_k,
                               const void* d_vec_v, int H_q, int H_kv, float scale,
                               float alpha_k, float alpha_v, float rope_base, hipStream_t stream) {
    if (!seqs || n_seq <= 0 || n_seq > 4096) return -100;
    if (H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || H_q / H_kv > 8) return -100;
    // The per-call argument block goes to the device with a copy from host
    // staging memory that the next call reuses: a captured copy would replay
    // whatever a later call left there, so capture is refused.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return -100;
    if (cap != hipStreamCaptureStatusNone) return -105;
    for (int i = 0; i < n_seq; i++) {
        const khq_seq& q = seqs[i];
        if (q.c_len < 0 || q.win_len < 0 || (q.c_len == 0 && q.win_len == 0)) return -100;
        if (q.win_len > 0 && (q.ring_cap <= 0 || q.win_len > q.ring_cap || q.win_start < 0))
            return -100;
    }
    const int n_rep = H_q / H_kv;
    bool batched = g_kernel_choice.load(std::memory_order_relaxed) == 0 && use_mfma(n_rep, H_kv, 1);
    for (int i = 0; i < n_seq && batched; i++) batched = seqs[i].win_len <= 256;
    if (!batched) {  // one fused step per sequence
        for (int i = 0; i < n_seq; i++) {
            const khq_seq& q = seqs[i];
            const int rc = khq_attn_step_fp16(
                q.q_gate, q.k_payload, q.v_payload, q.v_shared_meta, q.k_mask, q.k_norms,
                q.k_r_norms, q.v_norms, q.v_r_norms, centroids_k, centroids_v, vq_centroids,
                k_rotor, v_rotor, d_vec_k, d_vec_v, q.ring_k, q.ring_v, q.out, H_q, H_kv, q.c_len,
                q.win_start, q.win_len, q.ring_cap, scale, alpha_k, alpha_v, rope_base, stream);
            if (rc) return rc;
        }
        return 0;
    }
    // Chunk length: the smallest tile count per chunk whose compressed chunks
    // fit the CUs.  The window blocks (one per sequence with a window) are
    // dispatched first and are short; the chunk blocks follow longest first,
    // so the few that wait for a CU freed by a window block are the shortest.
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    std::vector<int> tiles(n_seq);
    long total_tiles = 0;
    int n_win = 0, max_tiles = 1;
    for (int i = 0; i < n_seq; i++) {
        tiles[i] = (seqs[i].c_len + 15) / 16;
        total_tiles += tiles[i];
        max_tiles = std::max(max_tiles, tiles[i]);
        n_win += seqs[i].win_len > 0 ? 1 : 0;
    }
    int per = std::max(1, (int)((total_tiles + cus - 1) / cus));
    auto chunks_for = [&](int p) {
        long b = 0;
        for (int i = 0; i < n_seq; i++) b += (tiles[i] + p - 1) / p;
        return b;
    };
    while (per < max_tiles && chunks_for(per) > cus) per++;
    auto blocks_for = [&](int p) { return chunks_for(p) + 4 * n_win; };
    // partial layout: sequence i owns H_q x np_i triples from float offset off_i
    static thread_local std::vector<khq::AttnArgs> h_args;
    static thread_local std::vector<khq::FinishArgs> h_fin;
    static thread_local std::vector<int2> h_map;
    h_args.assign(n_seq, khq::AttnArgs{});
    h_fin.assign(n_seq, khq::FinishArgs{});
    h_map.clear();
    size_t part_floats = 0;
    std::vector<size_t> off(n_seq);
    std::vector<int> chunks(n_seq), np(n_seq);
    // each sequence's chunks share its tiles evenly (at most per each): the
    // longest chunk sets the launch's length, so no sequence keeps one full
    // chunk and a short remainder
    std::vector<int> ctiles(n_seq);
    for (int i = 0; i < n_seq; i++) {
        chunks[i] = (tiles[i] + per - 1) / per;
        ctiles[i] = chunks[i] > 0 ? (tiles[i] + chunks[i] - 1) / chunks[i] : 1;
        np[i] = chunks[i] + (seqs[i].win_len > 0 ? 1 : 0);
        if (np[i] > 1024) return -100;  // finishing kernel's part limit
        off[i] = part_floats;
        part_floats += (size_t)H_q * np[i] * 258;
    }
    const size_t meta_off = (part_floats * sizeof(float) + 255) & ~(size_t)255;
    const size_t n_blocks = blocks_for(per);
    const size_t meta_bytes = n_seq * (sizeof(khq::AttnArgs) + sizeof(khq::FinishArgs)) +
                              n_blocks * sizeof(int2) + 512;
    float* ws = nullptr;
    hipError_t e = workspace(meta_off + meta_bytes, stream, &ws);
    if (e != hipSuccess) return rc_of(e);
    // metadata block (device and host staging share the layout): the
    // attention arguments, the finishing arguments, then the block map
    char* meta = reinterpret_cast<char*>(ws) + meta_off;
    const size_t o_fin = (n_seq * sizeof(khq::AttnArgs) + 15) & ~(size_t)15;
    const size_t o_map = (o_fin + n_seq * sizeof(khq::FinishArgs) + 15) & ~(size_t)15;
    khq::AttnArgs* d_args = reinterpret_cast<khq::AttnArgs*>(meta);
    khq::FinishArgs* d_fin = reinterpret_cast<khq::FinishArgs*>(meta + o_fin);
    int2* d_map = reinterpret_cast<int2*>(meta + o_map);
    for (int i = 0; i < n_seq; i++) {
        const khq_seq& q = seqs[i];
        khq::AttnArgs a = attn_args(q.q_gate, q.k_payload, q.v_payload, q.v_shared_meta, q.k_mask,
                                    q.k_norms, q.k_r_norms, q.v_norms, q.v_r_norms, centroids_k,
                                    centroids_v, vq_centroids, k_rotor, v_rotor, d_vec_k, d_vec_v);
        const int ring = q.ring_cap > 0 ? q.ring_cap : 1;
        a.part = ws + off[i];
        a.c_len = q.c_len;
        a.h_kv = H_kv;
        a.L_q = 1;
        a.start_pos = 0;
        a.n_parts = chunks[i];
        a.part_offset = 0;
        a.part_stride = np[i];
        a.sc = scale;
        a.a_k = alpha_k;
        a.a_v = alpha_v;
        a.rope_base = rope_base;
        a.ring_k = static_cast<const __half*>(q.ring_k);
        a.ring_v = static_cast<const __half*>(q.ring_v);
        a.win_start = q.win_start % ring;
        a.win_len = q.win_len;
        a.ring_cap = ring;
        a.win_blocks = 4;
        a.chunk_tiles = ctiles[i];
        khq::fill_rope_table(a);
        a.spin_limit = khq::g_spin_limit.load(std::memory_order_relaxed);
        h_args[i] = a;
        if (np[i] > chunks[i])  // window blocks, one per KV head
            for (int w = 0; w < 4; w++) h_map.push_back(int2{i, chunks[i] + w});
        khq::FinishArgs f{};
        f.part = ws + off[i];
        f.n_parts = np[i];
        f.part_stride = np[i];
        f.q = static_cast<const __half*>(q.q_gate);
        f.ring_k = a.ring_k;
        f.ring_v = a.ring_v;
        f.ring_cap = ring;
        f.win_start = a.win_start;
        f.win_len = 0;  // computed by the window blocks
        f.h_kv = H_kv;
        f.n_rep = n_rep;
        f.sc = scale;
        f.eps = 1e-8f;
        f.out = static_cast<__half*>(q.out);
        h_fin[i] = f;
    }
    {
        // chunk blocks after the window blocks, longest first
        std::vector<std::pair<int, int2>> cb;
        for (int i = 0; i < n_seq; i++)
            for (int c = 0; c < chunks[i]; c++)
                cb.push_back({std::min(ctiles[i], tiles[i] - c * ctiles[i]), int2{i, c}});
        std::stable_sort(cb.begin(), cb.end(),
                         [](const std::pair<int, int2>& x, const std::pair<int, int2>& y) {
                             return x.first > y.first;
                         });
        for (const auto& x : cb) h_map.push_back(x.second);
    }
    // one upload of the whole block from a pinned staging slot by a one-block
    // kernel that reads host memory: queued without waiting for the stream
    // (a pageable copy left ~17 us between consecutive calls, a DMA from the
    // pinned slot ~40 us).  Slots are reused round robin, each after the
    // event recorded behind the call that last used it.
    struct MetaSlot {
        char* host = nullptr;
        void* dev = nullptr;  // the slot's address for the GPU
        size_t cap = 0;
        hipEvent_t done = nullptr;
        bool pending = false;
    };
    static thread_local MetaSlot slots[4];
    static thread_local int next_slot = 0;
    MetaSlot& ms = slots[next_slot];
    next_slot = (next_slot + 1) & 3;
    const size_t n_meta = (o_map + h_map.size() * sizeof(int2) + 15) & ~(size_t)15;
    if (ms.pending) {
        e = hipEventSynchronize(ms.done);
        if (e != hipSuccess) return rc_of(e);
        ms.pending = false;
    }
    if (!ms.done) {
        e = hipEventCreateWithFlags(&ms.done, hipEventDisableTiming);
        if (e != hipSuccess) return rc_of(e);
    }
    if (ms.cap < n_meta) {
        if (ms.host) (void)hipHostFree(ms.host);
        ms.host = nullptr;
        ms.cap = 0;
        const size_t cap = (n_meta + 4095) & ~(size_t)4095;
        // coherent: the GPU reads the slot through the host link each time,
        // never from a cached copy of an earlier upload
        e = hipHostMalloc(reinterpret_cast<void**>(&ms.host), cap,
                          hipHostMallocMapped | hipHostMallocCoherent | hipHostMallocPortable);
        if (e != hipSuccess) return rc_of(e);
        e = hipHostGetDevicePointer(&ms.dev, ms.host, 0);
        if (e != hipSuccess) return rc_of(e);
        ms.cap = cap;
    }
    std::memcpy(ms.host, h_args.data(), n_seq * sizeof(khq::AttnArgs));
    std::memcpy(ms.host + o_fin, h_fin.data(), n_seq * sizeof(khq::FinishArgs));
    std::memcpy(ms.host + o_map, h_map.data(), h_map.size() * sizeof(int2));
    e = khq::launch_meta_upload(ms.dev, meta, n_meta, stream);
    if (e != hipSuccess) return rc_of(e);
    // from here on the upload may be reading the slot: every exit marks it
    // pending behind an event, so its reuse waits for the upload
    auto fail = [&](hipError_t err) {
        if (hipEventRecord(ms.done, stream) == hipSuccess) ms.pending = true;
        else (void)hipStreamSynchronize(stream);
        return rc_of(err);
    };
    e = khq::launch_attn_ws_batched(d_args, d_map, (int)h_map.size(), stream);
    if (e != hipSuccess) return fail(e);
    e = khq::launch_step_finish_batched(d_fin, n_seq, H_q, stream);
    if (e != hipSuccess) return fail(e);
    // behind the call's kernels (a marker between the upload and the
    // attention launch would delay the latter)
    e = hipEventRecord(ms.done, stream);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(stream);
        return rc_of(e);
    }
    ms.pending = true;
    return 0;
}

}  // extern "C"

namespace khq {

int prefill_attn_run(const __half* q_gate, const __half* k, const __half* vt, int ld_vt, int n_k,
                     int n_q, int vis0, int H_q, int H_kv, float scale, __half* out,
                     hipStream_t stream, int q_b, int hole_lo, int hole_hi, int ex_lo, int ex_hi,
                     bool merge) {
    if (n_k <= 0 || n_q <= 0 || vis0 < 1) return -100;
    if (q_b < 0 || q_b > n_q || hole_lo < 0 || hole_hi < hole_lo || hole_hi > n_k ||
        ex_hi < ex_lo || (ex_hi > ex_lo && ex_lo < n_k) ||
        (q_b > 0 && ex_hi - ex_lo != hole_hi - hole_lo))
        return -100;
    const int n_tot = std::max(n_k, ex_hi);
    // both attention kernels read V^T in 32-key tiles without a clamp, so the
    // leading dimension must cover the last tile
    if (H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 || ld_vt % 8 != 0 ||
        ld_vt < (n_tot + 31) / 32 * 32)
        return -100;
    const int n_rep = H_q / H_kv;
    int per = 0;
    const int ns = prefill_splits(n_q, n_rep, H_kv, n_tot, &per);
    float* ws = nullptr;
    hipError_t e = workspace((size_t)n_q * H_q * ns * 258 * sizeof(float), stream, &ws);
    if (e != hipSuccess) return rc_of(e);
    PrefillArgs a{};
    a.q = q_gate;
    a.k = k;
    a.vt = vt;
    a.part = ws;
    a.ld_vt = ld_vt;
    a.n_k = n_k;
    a.n_q = n_q;
    a.vis0 = vis0;
    a.h_kv = H_kv;
    a.n_rep = n_rep;
    a.n_split = ns;
    a.keys_per_split = per;
    a.sc = scale;
    a.n_tot = n_tot;
    a.q_b = q_b;
    a.hole_lo = hole_lo;
    a.hole_hi = hole_hi;
    a.ex_lo = ex_lo;
    a.ex_hi = ex_hi;
    e = launch_prefill_attn(a, stream);
    if (e != hipSuccess || !merge) return rc_of(e);
    return rc_of(launch_prefill_merge(ws, q_gate, out, n_q * H_q, ns, 1e-8f, stream));
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n == 0) {  // first query on this device: every caller computes the same value
        int v = 0;
        n = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v : 256;
        g_cu_count[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

hipError_t ensure_dynamic_lds(const void* kernel, int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    for (const LdsSet& x : g_lds_set)
        if (x.fn == kernel && x.dev == dev && x.bytes >= bytes) return hipSuccess;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
    g_lds_set.push_back(LdsSet{kernel, dev, bytes});
    return hipSuccess;
}

}  // namespace khq
