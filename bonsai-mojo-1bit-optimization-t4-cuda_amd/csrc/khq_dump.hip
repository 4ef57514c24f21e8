// khq_dump.hip -- calibration dumps of K/V activations and attention scores
// (the KHQD and KHQA files of ref:src/models/qwen3_5/khq_dump.mojo).
//
// KHQD, <dir>/kv_dump.bin (little-endian), written once by khq_dump_flush:
//   u32 'KHQD' | u32 n_layers | u32 dim
//   n_layers x (u32 layer_id | u32 n_tokens)            (layers in id order)
//   per layer: K rows (n_tokens x dim f32), then V rows (n_tokens x dim f32)
// KHQA, <dir>/attn_<layer>.bin, one record per dumped token:
//   u32 'KHQA' | u32 H_q | u32 H_kv | u32 D
//   per token: u32 n_valid (= pos + 1) | H_q x n_valid fp16 softmax scores
//
// The reference copies every token to the host with two synchronisations and
// computes the attention scores on the CPU.  Here the K/V rows accumulate in
// device memory (an asynchronous device-to-device copy per token, converted
// to f32 once at flush) and the scores of a token are computed on the GPU
// (one block per query head over the layer's roped-K history, fp32
// accumulate); only the finished fp16 record crosses to the host.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "khq.h"
#include "khq_internal.h"

namespace {

constexpr int kMaxLayers = 64;          // ref khq_dump.mojo:24
constexpr uint32_t kMagicKV = 0x4451484Bu;  // 'KHQD'
constexpr uint32_t kMagicAttn = 0x4151484Bu;  // 'KHQA'

// IEEE fp16 bits of v as the reference forms them (khq_dump.mojo:95-117):
// round to nearest even for normal results; subnormal results are
// round((512 + m / 16384) * 2^e) with halves rounded up, the reference's
// exp(e ln 2) taken as the exact power of two.
__device__ __forceinline__ uint16_t half_bits_ref(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const int ex = (int)((bits >> 23) & 0xFFu) - 127 + 15;
    const uint32_t man = bits & 0x7FFFFFu;
    if (ex >= 31) return sign | 0x7C00u;
    if (ex > 0) {
        uint16_t half = (uint16_t)(((uint32_t)ex << 10) | (man >> 13));
        const uint32_t rem = man & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
        return sign | half;
    }
    if (ex < -9) return sign;
    const float val16 = (512.0f + (float)man / 16384.0f) * ldexpf(1.0f, ex);
    return sign | (uint16_t)(uint32_t)(val16 + 0.5f);
}

// Scores of one token: block h = query head, threads over history rows.
// q_gate f16 [H_q][2 D] (q at 0..D-1), hist f16 [cap][H_kv * D] roped K.
constexpr int kThreads = 256;
__global__ __launch_bounds__(kThreads) void dump_scores_kernel(const __half* __restrict__ q_gate,
                                                               const __half* __restrict__ hist,
                                                               uint16_t* __restrict__ out,
                                                               int n_valid, int H_kv, int D,
                                                               int n_rep, float scale) {
    extern __shared__ float sm[];  // q [D], logits [n_valid], reduction [64]
    float* sq = sm;
    float* sl = sm + D;
    float* red = sl + n_valid;
    const int h = blockIdx.x, t = threadIdx.x, kv = h / n_rep;
    for (int d = t; d < D; d += kThreads) sq[d] = __half2float(q_gate[(size_t)h * 2 * D + d]);
    __syncthreads();
    float mx = -1e30f;
    for (int s = t; s < n_valid; s += kThreads) {
        const __half* kr = hist + ((size_t)s * H_kv + kv) * D;
        float acc = 0.0f;
        for (int d = 0; d < D; d++) acc = fmaf(sq[d], __half2float(kr[d]), acc);
        acc *= scale;
        sl[s] = acc;
        mx = fmaxf(mx, acc);
    }
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float z = 0.0f;
    for (int s = t; s < n_valid; s += kThreads) {
        const float e = expf(sl[s] - mx);
        sl[s] = e;
        z += e;
    }
    for (int o = 32; o >= 1; o >>= 1) z += __shfl_xor(z, o, 64);
    if ((t & 63) == 0) red[4 + (t >> 6)] = z;
    __syncthreads();
    z = (red[4] + red[5]) + (red[6] + red[7]);
    const float zinv = 1.0f / z;
    for (int s = t; s < n_valid; s += kThreads)
        out[(size_t)h * n_valid + s] = half_bits_ref(sl[s] * zinv);
}

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
    for (int i = 0; i < 4; i++) b.push_back((uint8_t)(v >> (8 * i)));
}

}  // namespace

struct khq_dump {
    std::string dir;
    int cap = 0, dim = 0, flags = 0;
    // KHQD: per layer fp16 K and V rows [cap][dim] on the device
    int n[kMaxLayers] = {0};
    __half* kbuf[kMaxLayers] = {nullptr};
    __half* vbuf[kMaxLayers] = {nullptr};
    // KHQA: per layer roped-K history [cap][dim], open files, score staging
    int H_q = 0, H_kv = 0, D = 0;
    __half* hist[kMaxLayers] = {nullptr};
    FILE* files[kMaxLayers] = {nullptr};
    uint16_t* d_scores = nullptr;
    uint16_t* h_scores = nullptr;  // pinned
    std::vector<uint8_t> rec;
};

namespace {

void dump_release(khq_dump* d) {
    for (int l = 0; l < kMaxLayers; l++) {
        if (d->kbuf[l]) (void)hipFree(d->kbuf[l]);
        if (d->vbuf[l]) (void)hipFree(d->vbuf[l]);
        if (d->hist[l]) (void)hipFree(d->hist[l]);
        if (d->files[l]) fclose(d->files[l]);
        d->kbuf[l] = d->vbuf[l] = d->hist[l] = nullptr;
        d->files[l] = nullptr;
    }
    if (d->d_scores) (void)hipFree(d->d_scores);
    if (d->h_scores) (void)hipHostFree(d->h_scores);
    d->d_scores = d->h_scores = nullptr;
}

}  // namespace

extern "C" {

khq_dump* khq_dump_create(const char* dir, int max_tokens, int kv_dim, int flags) {
    if (!dir || max_tokens <= 0 || kv_dim <= 0 || (flags & ~3) != 0 || flags == 0) return nullptr;
    khq_dump* d = new (std::nothrow) khq_dump();
    if (!d) return nullptr;
    d->dir = dir;
    d->cap = max_tokens;
    d->dim = kv_dim;
    d->flags = flags;
    return d;
}

void khq_dump_destroy(khq_dump* d) {
    if (!d) return;
    (void)hipDeviceSynchronize();
    dump_release(d);
    delete d;
}

int khq_dump_count(const khq_dump* d, int layer) {
    if (!d || layer < 0 || layer >= kMaxLayers) return -100;
    return d->n[layer];
}

int khq_dump_kv(khq_dump* d, int layer, const void* k, const void* v, hipStream_t stream) {
    if (!d || !k || !v) return -100;
    if (!(d->flags & KHQ_DUMP_KV) || layer < 0 || layer >= kMaxLayers) return 0;
    const int n = d->n[layer];
    if (n >= d->cap) return 0;  // full: further tokens are not recorded (ref :56-58)
    const size_t row = (size_t)d->dim * sizeof(__half);
    if (!d->kbuf[layer]) {
        if (hipMalloc(reinterpret_cast<void**>(&d->kbuf[layer]), row * d->cap) != hipSuccess)
            return (int)hipErrorOutOfMemory;
        if (hipMalloc(reinterpret_cast<void**>(&d->vbuf[layer]), row * d->cap) != hipSuccess) {
            (void)hipFree(d->kbuf[layer]);
            d->kbuf[layer] = nullptr;
            return (int)hipErrorOutOfMemory;
        }
    }
    hipError_t e = hipMemcpyAsync(d->kbuf[layer] + (size_t)n * d->dim, k, row,
                                  hipMemcpyDeviceToDevice, stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(d->vbuf[layer] + (size_t)n * d->dim, v, row, hipMemcpyDeviceToDevice,
                           stream);
    if (e != hipSuccess) return (int)e;
    d->n[layer] = n + 1;
    return 0;
}

int khq_dump_attn(khq_dump* d, int layer, const void* q_gate, const void* k_roped, int pos,
                  int H_q, int H_kv, int D, float scale, hipStream_t stream) {
    if (!d || !q_gate || !k_roped || pos < 0) return -100;
    if (!(d->flags & KHQ_DUMP_ATTN) || layer < 0 || layer >= kMaxLayers) return 0;
    if (pos >= d->cap) return 0;  // ref :207-208
    if (H_q <= 0 || H_kv <= 0 || D <= 0 || H_q % H_kv != 0 || H_kv * D != d->dim) return -100;
    if (d->H_q == 0) {  // the first call fixes the shape (ref :214-233)
        d->H_q = H_q;
        d->H_kv = H_kv;
        d->D = D;
        const size_t nb = (size_t)H_q * d->cap * sizeof(uint16_t);
        if (hipMalloc(reinterpret_cast<void**>(&d->d_scores), nb) != hipSuccess)
            return (int)hipErrorOutOfMemory;
        if (hipHostMalloc(reinterpret_cast<void**>(&d->h_scores), nb, hipHostMallocDefault) !=
            hipSuccess)
            return (int)hipErrorOutOfMemory;
    }
    if (H_q != d->H_q || H_kv != d->H_kv || D != d->D) return 0;  // ref :234-235
    const size_t row = (size_t)d->dim * sizeof(__half);
    if (!d->hist[layer]) {
        if (hipMalloc(reinterpret_cast<void**>(&d->hist[layer]), row * d->cap) != hipSuccess)
            return (int)hipErrorOutOfMemory;
        if (hipMemsetAsync(d->hist[layer], 0, row * d->cap, stream) != hipSuccess)
            return (int)hipErrorInvalidValue;
    }
    if (pos == 0) {  // a new sequence clears the history (ref :243-245)
        hipError_t e = hipMemsetAsync(d->hist[layer], 0, row * d->cap, stream);
        if (e != hipSuccess) return (int)e;
    }
    if (!d->files[layer]) {
        const std::string path = d->dir + "/attn_" + std::to_string(layer) + ".bin";
        FILE* f = fopen(path.c_str(), "wb");
        if (!f) return -104;
        std::vector<uint8_t> hdr;
        put_u32(hdr, kMagicAttn);
        put_u32(hdr, (uint32_t)H_q);
        put_u32(hdr, (uint32_t)H_kv);
        put_u32(hdr, (uint32_t)D);
        if (fwrite(hdr.data(), 1, hdr.size(), f) != hdr.size()) {
            fclose(f);
            return -104;
        }
        d->files[layer] = f;
    }
    hipError_t e = hipMemcpyAsync(d->hist[layer] + (size_t)pos * d->dim, k_roped, row,
                                  hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return (int)e;
    const int n_valid = pos + 1;
    const size_t smem = (size_t)(D + n_valid + 64) * sizeof(float);
    if (smem > 160 * 1024) return -100;  // histories up to ~40K tokens
    e = khq::ensure_dynamic_lds(reinterpret_cast<const void*>(&dump_scores_kernel), 160 * 1024);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(dump_scores_kernel, dim3(H_q), dim3(kThreads), smem, stream,
                       static_cast<const __half*>(q_gate), d->hist[layer], d->d_scores, n_valid,
                       H_kv, D, H_q / H_kv, scale);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const size_t nb = (size_t)H_q * n_valid * sizeof(uint16_t);
    e = hipMemcpyAsync(d->h_scores, d->d_scores, nb, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return (int)e;
    d->rec.clear();
    put_u32(d->rec, (uint32_t)n_valid);
    const size_t off = d->rec.size();
    d->rec.resize(off + nb);
    std::memcpy(d->rec.data() + off, d->h_scores, nb);
    if (fwrite(d->rec.data(), 1, d->rec.size(), d->files[layer]) != d->rec.size()) return -104;
    return 0;
}

int khq_dump_flush(khq_dump* d) {
    if (!d) return -100;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return (int)e;
    for (int l = 0; l < kMaxLayers; l++)
        if (d->files[l]) {
            fclose(d->files[l]);
            d->files[l] = nullptr;
        }
    if (!(d->flags & KHQ_DUMP_KV)) return 0;
    int n_layers = 0;
    for (int l = 0; l < kMaxLayers; l++) n_layers += d->n[l] > 0;
    if (n_layers == 0) return 0;  // nothing recorded: no file (ref :328-330)
    const std::string path = d->dir + "/kv_dump.bin";
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) return -104;
    std::vector<uint8_t> hdr;
    put_u32(hdr, kMagicKV);
    put_u32(hdr, (uint32_t)n_layers);
    put_u32(hdr, (uint32_t)d->dim);
    for (int l = 0; l < kMaxLayers; l++)
        if (d->n[l] > 0) {
            put_u32(hdr, (uint32_t)l);
            put_u32(hdr, (uint32_t)d->n[l]);
        }
    bool ok = fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
    std::vector<__half> h16;
    std::vector<float> f32;
    for (int l = 0; l < kMaxLayers && ok; l++) {
        const size_t cnt = (size_t)d->n[l] * d->dim;
        if (cnt == 0) continue;
        h16.resize(cnt);
        f32.resize(cnt);
        for (__half* src : {d->kbuf[l], d->vbuf[l]}) {
            if (hipMemcpy(h16.data(), src, cnt * sizeof(__half), hipMemcpyDeviceToHost) !=
                hipSuccess) {
                ok = false;
                break;
            }
            for (size_t i = 0; i < cnt; i++) f32[i] = __half2float(h16[i]);
            ok = fwrite(f32.data(), sizeof(float), cnt, f) == cnt;
            if (!ok) break;
        }
        d->n[l] = 0;  // the buffers are reused by a later recording
    }
    fclose(f);
    return ok ? 0 : -104;
}

}  // extern "C"
