// khq_finish.hip -- last stage of the fused two-region step: fp16 ring-window
// attention, logsumexp merge with the compressed-region partials, division by
// (den + eps) and the sigmoid gate, in one launch.
//
// One 256-thread block per (query head, 32-dim slice).  Every block of a head
// recomputes the window scores (win_len <= 256 rows of 512 B, which stay in
// L2) so no second launch is needed; each block then sums the window V and
// the compressed partials for its 32 dims only.  All global loads of a stage
// are issued before any of their values is used.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "khq_internal.h"
#include "khq_mfma_util.h"

namespace khq {
namespace fin {

using namespace mu;

typedef float f2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f2 ldg_f2(const float* p) {
    return *(const __attribute__((address_space(1))) f2*)p;
}
// Partial rows are 258 floats long, so a row's dims are only 8-byte aligned:
// they are read as 8-byte loads.

constexpr int DS = 32;         // dims per block
constexpr int MAX_WIN = 256;   // ring capacity bound
constexpr int MAX_PARTS = 1024;  // compressed partials (+ a window partial)

// Wavefront max / sum: rows of 16 by DPP, then xor 16 (swizzle) and xor 32.
__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    v = fmaxf(v, xor_lane<16>(v));
    return fmaxf(v, xor_lane<32>(v));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += xor_lane<16>(v);
    return v + xor_lane<32>(v);
}

// Block-wide max of (x, y) in one pass; s_red holds 8 floats.
__device__ __forceinline__ void block_max2(float& x, float& y, float* s_red) {
    x = wave_max(x);
    y = wave_max(y);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        s_red[threadIdx.x >> 6] = x;
        s_red[4 + (threadIdx.x >> 6)] = y;
    }
    __syncthreads();
    x = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    y = fmaxf(fmaxf(s_red[4], s_red[5]), fmaxf(s_red[6], s_red[7]));
}
__device__ __forceinline__ void block_sum2(float& x, float& y, float* s_red) {
    x = wave_sum(x);
    y = wave_sum(y);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        s_red[threadIdx.x >> 6] = x;
        s_red[4 + (threadIdx.x >> 6)] = y;
    }
    __syncthreads();
    x = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    y = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);
}

__device__ __forceinline__ void finish_block(const FinishArgs& a, int hq, int slice) {
    __shared__ float s_p[MAX_WIN];      // window weights
    __shared__ float s_w[MAX_PARTS];    // compressed part weights
    __shared__ float s_red[8];
    __shared__ float s_acc[2][8][DS];
    const int t = threadIdx.x;
    const int d0 = slice * DS;
    const int hk = hq / a.n_rep;
    const float* base = a.part + (size_t)hq * a.part_stride * 258;  // < 2^31 floats per head
    const int d = t & (DS - 1), grp = t >> 5;
    const int np = a.n_parts, wl = a.win_len;
    const int last_p = max(np - 1, 0), last_w = max(wl - 1, 0);
    const int cap = a.ring_cap;  // win_start < cap and win_len <= cap (host-checked)
    auto slot_of = [&](int s) {
        const int x = a.win_start + s;
        return x >= cap ? x - cap : x;
    };

    // ---- every load of the block is issued here, from clamped indices
    float mcv[MAX_PARTS / 256], lcv[MAX_PARTS / 256];
#pragma unroll
    for (int k = 0; k < MAX_PARTS / 256; k++) {
        const float* pp = base + (size_t)min(t + 256 * k, last_p) * 258;
        mcv[k] = pp[256];
        lcv[k] = pp[257];
    }
    float pacc[32];  // parts grp + 8 u (first 256 parts)
#pragma unroll
    for (int u = 0; u < 32; u++) pacc[u] = base[min(grp + 8 * u, last_p) * 258 + d0 + d];
    __half vw[32];   // window rows grp + 8 u
#pragma unroll
    for (int u = 0; u < 32; u++) vw[u] = __ushort_as_half((unsigned short)0);
    if (wl > 0) {
#pragma unroll
        for (int u = 0; u < 32; u++) {
            const int slot = slot_of(min(grp + 8 * u, last_w));
            vw[u] = a.ring_v[(slot * a.h_kv + hk) * 256 + d0 + d];
        }
    }
    const int sub = t >> 4, l16 = t & 15;
    const __half* qrow = a.q + (size_t)hq * 512 + 16 * l16;
    const h8 qa = __builtin_bit_cast(h8, reinterpret_cast<const uint4*>(qrow)[0]);
    const h8 qb = __builtin_bit_cast(h8, reinterpret_cast<const uint4*>(qrow)[1]);
    const float gate = __half2float(a.q[(size_t)hq * 512 + 256 + d0 + (t & (DS - 1))]);

    // ---- window scores: 16 threads per row (16 dims each), 16 rows per round
    float wmax = -1e20f;
    const int n_rounds = (wl + 15) / 16;
    for (int r0 = 0; r0 < n_rounds; r0 += 8) {
        uint4 kr[8][2];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int slot = slot_of(min(16 * (r0 + u) + sub, last_w));
            const uint4* kp = reinterpret_cast<const uint4*>(
                a.ring_k + (slot * a.h_kv + hk) * 256 + 16 * l16);
            kr[u][0] = kp[0];
            kr[u][1] = kp[1];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const h8 ka = __builtin_bit_cast(h8, kr[u][0]), kb = __builtin_bit_cast(h8, kr[u][1]);
            float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                x0 = fmaf((float)qa[e], (float)ka[e], x0);
                x1 = fmaf((float)qb[e], (float)kb[e], x1);
            }
            const float dot = row16_sum(x0 + x1);
            const int s = 16 * (r0 + u) + sub;
            if (s < wl) {
                const float sc = dot * a.sc;
                if (l16 == 0) s_p[s] = sc;
                wmax = fmaxf(wmax, sc);
            }
        }
    }
    float mcmax = -1e20f;
#pragma unroll
    for (int k = 0; k < MAX_PARTS / 256; k++)
        if (t + 256 * k < np) mcmax = fmaxf(mcmax, mcv[k]);
    float Mw = wmax, Mc = mcmax;
    block_max2(Mw, Mc, s_red);

    // ---- weights: window exp(s - Mw), parts exp(m - Mc); zero past the ends,
    // so the sums below need no bounds (clamped loads hold finite values)
    float lw = 0.0f, lc = 0.0f;
    {
        const float p = t < wl ? expf(s_p[t] - Mw) : 0.0f;
        s_p[t] = p;
        lw = p;
    }
#pragma unroll
    for (int k = 0; k < MAX_PARTS / 256; k++) {
        const int s = t + 256 * k;
        const float wgt = s < np ? expf(mcv[k] - Mc) : 0.0f;
        s_w[s] = wgt;
        lc = fmaf(s < np ? lcv[k] : 0.0f, wgt, lc);
    }
    float Lw = lw, Lc = lc;
    block_sum2(Lw, Lc, s_red);  // its barriers also publish s_p / s_w

    // ---- numerators for dims d0 + d: rows / parts strided by the 8 groups
    float aw[4] = {0.f, 0.f, 0.f, 0.f}, ac[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 32; u++) {
        const int s = grp + 8 * u;
        aw[u & 3] = fmaf(s_p[s], __half2float(vw[u]), aw[u & 3]);
        ac[u & 3] = fmaf(s_w[s], pacc[u], ac[u & 3]);
    }
    for (int s = grp + 256; s < np; s += 8)  // parts beyond the first 256
        ac[0] = fmaf(s_w[s], base[(size_t)s * 258 + d0 + d], ac[0]);
    s_acc[0][grp][d] = (aw[0] + aw[1]) + (aw[2] + aw[3]);
    s_acc[1][grp][d] = (ac[0] + ac[1]) + (ac[2] + ac[3]);
    __syncthreads();
    if (t < DS) {
        float nw = 0.0f, nc = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            nw += s_acc[0][g][t];
            nc += s_acc[1][g][t];
        }
        const float M = fmaxf(Mw, Mc);
        const float fw = wl > 0 ? expf(Mw - M) : 0.0f;
        const float fc = np > 0 ? expf(Mc - M) : 0.0f;
        const float num = fmaf(nc, fc, nw * fw);
        const float den = fmaf(Lc, fc, Lw * fw);
        float val = num / (den + a.eps);
        val = val * (1.0f / (1.0f + expf(-gate)));
        a.out[(size_t)hq * 256 + d0 + t] = __float2half(val);
    }
}

__global__ __launch_bounds__(256) void step_finish_kernel(FinishArgs a) {
    finish_block(a, blockIdx.x, blockIdx.y);
}

// Global-memory load through a pointer read from memory (keeps the access a
// global load instead of a flat one).
template <typename T>
__device__ __forceinline__ T gload(const T* p) {
    return *(const __attribute__((address_space(1))) T*)p;
}

// Batched form (window computed upstream, a few parts per sequence): one
// block per (sequence, query head), thread = dim; each thread walks the
// row's parts (the (m, l) pairs are the same addresses for the whole block),
// 8 parts' loads in flight at a time.
__global__ __launch_bounds__(256) void step_finish_batched_kernel(const FinishArgs* __restrict__ args,
                                                                  int H_q) {
    const FinishArgs& a = args[blockIdx.x / H_q];
    const int hq = blockIdx.x % H_q, d = threadIdx.x;
    const float* base = a.part + (size_t)hq * a.part_stride * 258;
    const int np = a.n_parts;
    float M = -1e30f;
    for (int p0 = 0; p0 < np; p0 += 8) {
        float mv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) mv[i] = gload(base + (size_t)min(p0 + i, np - 1) * 258 + 256);
#pragma unroll
        for (int i = 0; i < 8; i++) M = fmaxf(M, mv[i]);
    }
    float num = 0.0f, den = 0.0f;
    for (int p0 = 0; p0 < np; p0 += 8) {
        float av[8], mv[8], lv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float* pp = base + (size_t)min(p0 + i, np - 1) * 258;
            av[i] = gload(pp + d);
            mv[i] = gload(pp + 256);
            lv[i] = gload(pp + 257);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float w = p0 + i < np ? __expf(mv[i] - M) : 0.0f;
            num = fmaf(av[i], w, num);
            den = fmaf(lv[i], w, den);
        }
    }
    const unsigned short gb =
        gload(reinterpret_cast<const unsigned short*>(a.q) + (size_t)hq * 512 + 256 + d);
    const float g = __half2float(__ushort_as_half(gb));
    const float val = num / (den + a.eps) * (1.0f / (1.0f + expf(-g)));
    *(__attribute__((address_space(1))) unsigned short*)(reinterpret_cast<unsigned short*>(a.out) +
                                                          (size_t)hq * 256 + d) =
        __half_as_ushort(__float2half(val));
}

// Merge-only form (the window is already a part): one 256-thread block per
// (query head, 32-dim slice).  Lane l of wavefront w reads dims
// d0 + 4 (l % 8) .. + 3 of part 64 w + 8 i + l / 8 (i = 0..7), so one load
// instruction covers eight part rows, 128 contiguous bytes each, instead of
// 64 rows at 8 bytes a lane.  The head's maximum crosses the wavefronts
// through LDS; numerators and denominators sum over the eight part lanes
// (xor 8 / 16 / 32), then over the four wavefronts.  For n_parts <= 256
// every load is issued before the first value is used.
__device__ __forceinline__ f2 ld_ml(const float* pp) { return ldg_f2(pp + 256); }

__global__ __launch_bounds__(256) void step_merge_kernel(FinishArgs a) {
    __shared__ float s_m[4], s_den[4];
    __shared__ f4 s_num[4][8];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int sub = lane >> 3, c = lane & 7;
    const int hq = blockIdx.x;
    const int d = blockIdx.y * 32 + 4 * c;
    const float* base = a.part + (size_t)hq * a.part_stride * 258;
    const int np = a.n_parts, last = max(np - 1, 0);
    f4 num = f4{0.f, 0.f, 0.f, 0.f};
    float den = 0.0f;
    auto block_max = [&](float m) {
        m = wave_max(m);
        if (lane == 0) s_m[w] = m;
        __syncthreads();
        return fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    };
    if (np <= 256) {
        f2 ml[8], o[8][2];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float* pp = base + (size_t)min(64 * w + 8 * i + sub, last) * 258;
            ml[i] = ld_ml(pp);
            o[i][0] = ldg_f2(pp + d);
            o[i][1] = ldg_f2(pp + d + 2);
        }
        float m = -3.0e38f;
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (64 * w + 8 * i + sub < np) m = fmaxf(m, ml[i].x);
        const float M = block_max(m);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float wt = 64 * w + 8 * i + sub < np ? __expf(ml[i].x - M) : 0.0f;
            den = fmaf(ml[i].y, wt, den);
            num[0] = fmaf(o[i][0].x, wt, num[0]);
            num[1] = fmaf(o[i][0].y, wt, num[1]);
            num[2] = fmaf(o[i][1].x, wt, num[2]);
            num[3] = fmaf(o[i][1].y, wt, num[3]);
        }
    } else {
        float m = -3.0e38f;
        for (int p = t; p < np; p += 256) m = fmaxf(m, base[(size_t)p * 258 + 256]);
        const float M = block_max(m);
        for (int p = 64 * w + sub; p < np; p += 256)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int q = p + 8 * i;
                if (q < np) {
                    const float* pp = base + (size_t)q * 258;
                    const f2 mq = ld_ml(pp), o0 = ldg_f2(pp + d), o1 = ldg_f2(pp + d + 2);
                    const float wt = __expf(mq.x - M);
                    den = fmaf(mq.y, wt, den);
                    num[0] = fmaf(o0.x, wt, num[0]);
                    num[1] = fmaf(o0.y, wt, num[1]);
                    num[2] = fmaf(o1.x, wt, num[2]);
                    num[3] = fmaf(o1.y, wt, num[3]);
                }
            }
    }
    // sum over the eight part lanes of each dim group
#pragma unroll
    for (int j = 0; j < 4; j++) {
        num[j] += xor_lane<8>(num[j]);
        num[j] += xor_lane<16>(num[j]);
        num[j] += xor_lane<32>(num[j]);
    }
    den += xor_lane<8>(den);
    den += xor_lane<16>(den);
    den += xor_lane<32>(den);
    if (lane < 8) s_num[w][c] = num;
    if (lane == 0) s_den[w] = den;
    __syncthreads();
    if (t < 32) {
        const int g = t >> 2, j = t & 3;
        const float v = (s_num[0][g][j] + s_num[1][g][j]) + (s_num[2][g][j] + s_num[3][g][j]);
        const float D = (s_den[0] + s_den[1]) + (s_den[2] + s_den[3]);
        const int dd = blockIdx.y * 32 + t;
        const float gt = __half2float(a.q[(size_t)hq * 512 + 256 + dd]);
        const float val = v / (D + a.eps) * (1.0f / (1.0f + expf(-gt)));
        a.out[(size_t)hq * 256 + dd] = __float2half(val);
    }
}

}  // namespace fin

// Upload of a metadata block from pinned host memory by the GPU itself
// (16-byte loads over the host link, one per thread, so the whole block is a
// single round trip): it runs in stream order like a copy, but the host call
// that queues it returns at once.
__global__ __launch_bounds__(256) void meta_upload_kernel(const uint4* __restrict__ src,
                                                          uint4* __restrict__ dst, int n16) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

hipError_t launch_meta_upload(const void* host_src, void* dst, size_t bytes, hipStream_t st) {
    if (bytes % 16 != 0) return hipErrorInvalidValue;
    const int n16 = (int)(bytes / 16);
    hipLaunchKernelGGL(meta_upload_kernel, dim3((n16 + 255) / 256), dim3(256), 0, st,
                       static_cast<const uint4*>(host_src), static_cast<uint4*>(dst), n16);
    return hipGetLastError();
}

hipError_t launch_step_finish_batched(const FinishArgs* args, int n_seq, int H_q,
                                      hipStream_t st) {
    hipLaunchKernelGGL(fin::step_finish_batched_kernel, dim3(n_seq * H_q), dim3(256), 0, st, args,
                       H_q);
    return hipGetLastError();
}

hipError_t launch_step_finish(const FinishArgs& a, int H_q, hipStream_t st) {
    if (a.n_parts > fin::MAX_PARTS || a.win_len > fin::MAX_WIN || a.n_rep <= 0)
        return hipErrorInvalidValue;
    if (a.win_len == 0 && a.n_parts > 0) {
        hipLaunchKernelGGL(fin::step_merge_kernel, dim3(H_q, 8), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(fin::step_finish_kernel, dim3(H_q, 256 / fin::DS), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace khq
