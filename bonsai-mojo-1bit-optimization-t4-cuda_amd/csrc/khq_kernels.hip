// khq_kernels.hip -- KHQ compressed-KV decode attention for MI355X (gfx950).
//
// Kernels are written for 64-lane wavefronts.  The common lane mapping is
// "lane p owns patch p": dims 4p..4p+3 of a 256-wide head, so one wavefront
// covers one head row and the 4x4 per-patch rotors never leave a lane.
// The 256-point Walsh-Hadamard transform is then two in-lane butterfly
// stages followed by six cross-lane stages (lane xor 1..32).
//
// Compiled with -ffp-contract=off: every fused multiply-add is an explicit
// fmaf(), so the compress kernel reproduces the CPU restatement's operation
// sequence bit for bit.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "khq_internal.h"
#include "khq_compress_row.h"

namespace khq {

__global__ __launch_bounds__(256) void compress_kernel(
    const __half* __restrict__ x, const __half* __restrict__ d_vec,
    const __half* __restrict__ rotor, const __half* __restrict__ cents,
    const __half* __restrict__ vq, uint32_t* __restrict__ out_mask,
    __half* __restrict__ out_norms, __half* __restrict__ out_rn,
    uint8_t* __restrict__ out_pay, uint8_t* __restrict__ out_sm, int n, float ts,
    float alpha, int is_v) {
    compress_block(x, d_vec, rotor, cents, vq, out_mask, out_norms, out_rn, out_pay, out_sm, n, ts,
                   alpha, is_v, (int)blockIdx.x);
}

// K and V of one compression event in one launch: blocks [0, nb_k) run the K
// rows, the rest the V rows (the K job's shared-meta word, which the V job
// sets, is not written).
__global__ __launch_bounds__(256) void compress_pair_kernel(CompressJob k, CompressJob v,
                                                            int nb_k) {
    if ((int)blockIdx.x < nb_k)
        compress_block(k.x, k.d_vec, k.rotor, k.cents, k.vq, k.out_mask, k.out_norms, k.out_rn,
                       k.out_pay, nullptr, k.n, k.ts, k.alpha, 0, (int)blockIdx.x);
    else
        compress_block(v.x, v.d_vec, v.rotor, v.cents, v.vq, v.out_mask, v.out_norms, v.out_rn,
                       v.out_pay, v.out_sm, v.n, v.ts, v.alpha, 1, (int)blockIdx.x - nb_k);
}

// ------------------------------------------------- compressed-region parts
// One 256-thread block per (token part, KV head, query position).  Each of
// the four wavefronts walks every fourth token of the part; per token the
// packed K row is decoded ONCE and shared by the n_rep query heads of the
// KV group (the reference decodes it once per query head).  V is
// accumulated in the rotated domain and the inverse rotor + FWHT + 1/(16 d_v)
// are applied once per part after the four wavefronts are merged.
template <int NREP>
__global__ __launch_bounds__(256) void attn_part_kernel(AttnArgs a) {
    __shared__ float s_acc[4][NREP][256];
    __shared__ float s_ml[4][NREP][2];
    const int wave = threadIdx.x >> 6;
    const int p = threadIdx.x & 63;  // patch
    const int part = blockIdx.x;
    const int hkv = blockIdx.y;
    const int l_idx = blockIdx.z;
    const int s_limit = (a.L_q > 1) ? min(a.c_len, l_idx + 1) : a.c_len;
    const int per = (s_limit + a.n_parts - 1) / a.n_parts;
    const int lo = min(part * per, s_limit);
    const int hi = min(lo + per, s_limit);

    // per-lane constants
    float q[NREP][4];
#pragma unroll
    for (int i = 0; i < NREP; i++) {
        const int h = hkv * NREP + i;
        const __half* qp = a.q + (size_t)h * 512 + p * 4;
#pragma unroll
        for (int c = 0; c < 4; c++) q[i][c] = h2f(qp[c]);
    }
    float rk[16];
#pragma unroll
    for (int t = 0; t < 16; t++) rk[t] = h2f(a.rotor_k[p * 16 + t]);
    float cbk[4], dks[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        cbk[c] = h2f(a.cents_k[512 + p * 4 + c]);
        dks[c] = (1.0f / 256.0f) / (h2f(a.dk[p * 4 + c]) + 1e-8f);
    }
    const float cv0 = h2f(a.cents_v[p * 4 + 3]) * a.a_v;
    const float cv1 = h2f(a.cents_v[256 + p * 4 + 3]) * a.a_v;
    const __half* vcb = a.vq + (size_t)p * 768;

    // RoPE on dims 0..63 (lanes 0..15); pair (i, i+32) = lanes p, p^8
    const bool rope_lane = p < 16;
    float freq[4], cc[4], ss[4], stc[4], sts[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int m = (p * 4 + c) & 31;
        freq[c] = powf(a.rope_base, -2.0f * (float)m / 64.0f);
        stc[c] = cosf(4.0f * freq[c]);
        sts[c] = sinf(4.0f * freq[c]);
        cc[c] = 1.0f;
        ss[c] = 0.0f;
    }

    float acc[NREP][4];
    float mx[NREP], sm[NREP];
#pragma unroll
    for (int i = 0; i < NREP; i++) {
        mx[i] = -1e20f;
        sm[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) acc[i][c] = 0.0f;
    }

    const uint64_t lt = lanemask_lt();
    int since_anchor = 1 << 30;
    for (int s = lo + wave; s < hi; s += 4) {
        if (since_anchor >= 64) {  // exact angle every 256 tokens
            if (rope_lane) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float th = (float)(a.start_pos + s) * freq[c];
                    cc[c] = cosf(th);
                    ss[c] = sinf(th);
                }
            }
            since_anchor = 0;
        }
        const size_t g = (size_t)s * a.h_kv + hkv;
        // ---- K decode
        const uint8_t* kb = a.kpay + g * 40;
        const unsigned mword = *reinterpret_cast<const uint32_t*>(kb);
        float mult = (float)mword / 1000.0f;
        if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
        const float nk = h2f(a.knorm[g]);
        const float rs = h2f(a.krn[g]);
        const unsigned mb = reinterpret_cast<const uint8_t*>(a.kmask + g * 16)[p];
        unsigned code[4];
        unsigned base = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            code[c] = (mb >> (2 * c)) & 3u;
            base += (unsigned)__popcll(__ballot(code[c] == 3u) & lt);
        }
        float kv[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float cbase = cbk[c] * mult;
            float v = 0.0f;
            if (code[c] == 3u) {
                const unsigned j = base;
                float sign = -1.0f, r4 = 0.0f;
                if (j < 50u) {
                    sign = ((kb[29 + j / 8] >> (j % 8)) & 1u) ? 1.0f : -1.0f;
                    r4 = (float)((kb[4 + j / 2] >> ((j % 2) * 4)) & 0xFu);
                }
                v = sign * fmaf(r4, rs, cbase);
                base++;
            } else if (code[c] == 2u) {
                v = cbase;
            } else if (code[c] == 1u) {
                v = -cbase;
            }
            kv[c] = v * a.a_k * nk;
        }
        float k[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float t = kv[0] * rk[c * 4 + 0];
            t = fmaf(kv[1], rk[c * 4 + 1], t);
            t = fmaf(kv[2], rk[c * 4 + 2], t);
            t = fmaf(kv[3], rk[c * 4 + 3], t);
            k[c] = t;
        }
        fwht256(k);
#pragma unroll
        for (int c = 0; c < 4; c++) k[c] *= dks[c];
        {
            float xo[4];
#pragma unroll
            for (int c = 0; c < 4; c++) xo[c] = __shfl_xor(k[c], 8, 64);
            if (rope_lane) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    if (p < 8) k[c] = fmaf(k[c], cc[c], -(xo[c] * ss[c]));
                    else k[c] = fmaf(xo[c], ss[c], k[c] * cc[c]);
                    const float nc = fmaf(cc[c], stc[c], -(ss[c] * sts[c]));
                    const float ns = fmaf(ss[c], stc[c], cc[c] * sts[c]);
                    cc[c] = nc;
                    ss[c] = ns;
                }
            }
        }
        since_anchor++;
        // ---- scores for the n_rep heads of the group
        float sc[NREP];
#pragma unroll
        for (int i = 0; i < NREP; i++) {
            float t = q[i][0] * k[0];
            t = fmaf(q[i][1], k[1], t);
            t = fmaf(q[i][2], k[2], t);
            t = fmaf(q[i][3], k[3], t);
            sc[i] = wave_sum(t) * a.sc;
        }
        // ---- V decode (rotated domain)
        const uint8_t* vb = a.vpay + g * 104;
        const uint32_t* vw = reinterpret_cast<const uint32_t*>(vb);
        const unsigned grp = (unsigned)p >> 3, sub = (unsigned)p & 7u;
        const uint64_t w0 = vw[grp * 3 + 0], w1 = vw[grp * 3 + 1], w2 = vw[grp * 3 + 2];
        const uint64_t low64 = (w1 << 32) | w0;
        const uint64_t high64 = (w2 << 32) | w1;
        const unsigned pvl = (sub < 4) ? (unsigned)((low64 >> (sub * 12)) & 0xFFFu)
                                       : (unsigned)((high64 >> ((sub - 4) * 12 + 16)) & 0xFFFu);
        const unsigned hw = vw[24 + (p >> 5)];
        const unsigned vcode = (pvl & 0x7Fu) | (((hw >> (p & 31)) & 1u) << 7);
        const unsigned d3c = (pvl >> 7) & 1u;
        const unsigned d3d = (pvl >> 8) & 0xFu;
        const float nv = h2f(a.vnorm[g]);
        const float ec = h2f(a.vrn[g]);
        const float smv = *reinterpret_cast<const float*>(a.vsm + g * 4);
        const float pre_v = (a.a_v * nv) * ec;
        const float pre_r = smv * nv;
        float vv[4];
        vv[0] = h2f(vcb[vcode * 3 + 0]) * pre_v;
        vv[1] = h2f(vcb[vcode * 3 + 1]) * pre_v;
        vv[2] = h2f(vcb[vcode * 3 + 2]) * pre_v;
        vv[3] = fmaf(((float)d3d - 8.0f) / 7.0f, pre_r, (d3c ? cv1 : cv0) * nv);
        // ---- online softmax + accumulate
#pragma unroll
        for (int i = 0; i < NREP; i++) {
            float e;
            if (sc[i] > mx[i]) {
                const float fac = expf(mx[i] - sc[i]);
                sm[i] = fmaf(sm[i], fac, 1.0f);
#pragma unroll
                for (int c = 0; c < 4; c++) acc[i][c] *= fac;
                mx[i] = sc[i];
                e = 1.0f;
            } else {
                e = expf(sc[i] - mx[i]);
                sm[i] += e;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) acc[i][c] = fmaf(e, vv[c], acc[i][c]);
        }
    }

    // ---- merge the four wavefronts
#pragma unroll
    for (int i = 0; i < NREP; i++) {
#pragma unroll
        for (int c = 0; c < 4; c++) s_acc[wave][i][p * 4 + c] = acc[i][c];
        if (p == 0) {
            s_ml[wave][i][0] = mx[i];
            s_ml[wave][i][1] = sm[i];
        }
    }
    __syncthreads();
    for (int i = wave; i < NREP; i += 4) {
        float M = -1e20f;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, s_ml[w][i][0]);
        float den = 0.0f;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = expf(s_ml[w][i][0] - M);
            den = fmaf(s_ml[w][i][1], f, den);
#pragma unroll
            for (int c = 0; c < 4; c++) o[c] = fmaf(s_acc[w][i][p * 4 + c], f, o[c]);
        }
        // inverse V rotor + FWHT + (1/16)/d_v, ref .cu:1776-1826
        const __half* R = a.rotor_v + p * 16;
        float t[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float u = o[0] * h2f(R[c * 4 + 0]);
            u = fmaf(o[1], h2f(R[c * 4 + 1]), u);
            u = fmaf(o[2], h2f(R[c * 4 + 2]), u);
            u = fmaf(o[3], h2f(R[c * 4 + 3]), u);
            t[c] = u;
        }
        fwht256(t);
        const int h = hkv * NREP + i;
        const int qid = h * a.L_q + l_idx;
        float* out = a.part + ((size_t)qid * a.part_stride + a.part_offset + part) * 258;
#pragma unroll
        for (int c = 0; c < 4; c++)
            out[p * 4 + c] = (t[c] * (1.0f / 16.0f)) / (h2f(a.dv[p * 4 + c]) + 1e-8f);
        if (p == 0) {
            out[256] = M;
            out[257] = den;
        }
    }
}

// --------------------------------------------------------- fp16 window parts
// One 256-thread block per (window part, KV head); each wavefront walks every
// fourth slot of the part, lane p holding dims 4p..4p+3 of K and V, and the
// n_rep heads of the group share each K/V row.
template <int NREP>
__global__ __launch_bounds__(256) void window_part_kernel(WinArgs a) {
    __shared__ float s_acc[4][NREP][256];
    __shared__ float s_ml[4][NREP][2];
    const int wave = threadIdx.x >> 6;
    const int p = threadIdx.x & 63;
    const int part = blockIdx.x;
    const int hkv = blockIdx.y;
    const int per = (a.win_len + a.n_parts - 1) / a.n_parts;
    const int lo = min(part * per, a.win_len);
    const int hi = min(lo + per, a.win_len);
    float q[NREP][4];
#pragma unroll
    for (int i = 0; i < NREP; i++) {
        const __half* qp = a.q + (size_t)(hkv * NREP + i) * 512 + p * 4;
#pragma unroll
        for (int c = 0; c < 4; c++) q[i][c] = h2f(qp[c]);
    }
    float acc[NREP][4], mx[NREP], sm[NREP];
#pragma unroll
    for (int i = 0; i < NREP; i++) {
        mx[i] = -1e20f;
        sm[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) acc[i][c] = 0.0f;
    }
    // the wavefront's slots lo + wave + 4 j in groups of WG, every load of a
    // group issued before the first is used (same slot order as one at a time)
    constexpr int WG = 4;
    for (int s0 = lo + wave; s0 < hi; s0 += 4 * WG) {
        uint2 kraw[WG], vraw[WG];
#pragma unroll
        for (int j = 0; j < WG; j++) {
            const int s = min(s0 + 4 * j, hi - 1);
            const int slot = (a.win_start + s) % a.ring_cap;
            const size_t off = ((size_t)slot * a.h_kv + hkv) * 256 + p * 4;
            kraw[j] = *reinterpret_cast<const uint2*>(a.ring_k + off);
            vraw[j] = *reinterpret_cast<const uint2*>(a.ring_v + off);
        }
#pragma unroll
        for (int j = 0; j < WG; j++) {
            if (s0 + 4 * j >= hi) break;  // uniform per wavefront
            const __half* kh = reinterpret_cast<const __half*>(&kraw[j]);
            const __half* vh = reinterpret_cast<const __half*>(&vraw[j]);
            float k[4], v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) { k[c] = h2f(kh[c]); v[c] = h2f(vh[c]); }
#pragma unroll
            for (int i = 0; i < NREP; i++) {
                float t = q[i][0] * k[0];
                t = fmaf(q[i][1], k[1], t);
                t = fmaf(q[i][2], k[2], t);
                t = fmaf(q[i][3], k[3], t);
                const float sv = wave_sum(t) * a.sc;
                float e;
                if (sv > mx[i]) {
                    const float fac = expf(mx[i] - sv);
                    sm[i] = fmaf(sm[i], fac, 1.0f);
#pragma unroll
                    for (int c = 0; c < 4; c++) acc[i][c] *= fac;
                    mx[i] = sv;
                    e = 1.0f;
                } else {
                    e = expf(sv - mx[i]);
                    sm[i] += e;
                }
#pragma unroll
                for (int c = 0; c < 4; c++) acc[i][c] = fmaf(e, v[c], acc[i][c]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NREP; i++) {
#pragma unroll
        for (int c = 0; c < 4; c++) s_acc[wave][i][p * 4 + c] = acc[i][c];
        if (p == 0) {
            s_ml[wave][i][0] = mx[i];
            s_ml[wave][i][1] = sm[i];
        }
    }
    __syncthreads();
    for (int i = wave; i < NREP; i += 4) {
        float M = -1e20f;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, s_ml[w][i][0]);
        float den = 0.0f, o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = expf(s_ml[w][i][0] - M);
            den = fmaf(s_ml[w][i][1], f, den);
#pragma unroll
            for (int c = 0; c < 4; c++) o[c] = fmaf(s_acc[w][i][p * 4 + c], f, o[c]);
        }
        const int h = hkv * NREP + i;
        float* out = a.part + ((size_t)h * a.part_stride + a.part_offset + part) * 258;
#pragma unroll
        for (int c = 0; c < 4; c++) out[p * 4 + c] = o[c];
        if (p == 0) {
            out[256] = M;
            out[257] = den;
        }
    }
}

// ------------------------------------------------------ logsumexp combines
// Unnormalised merge of n_parts partial triples per query (the reduce of
// ref .cu:1836-1877).  Block (query, 64-dim slice): the 256 threads first
// find the maximum and the per-part weights exp(m_s - M) cooperatively
// (weights kept in LDS), then 4 groups of 64 threads sum disjoint part
// ranges for the 64 dims and the groups are added in LDS.
constexpr int kMaxParts = 4096;

__device__ __forceinline__ void lse_weights(const float* base, int n_parts, float* s_w,
                                            float* s_red, float& M, float& den) {
    const int t = threadIdx.x;
    float m = -1e20f;
    for (int s = t; s < n_parts; s += 256) m = fmaxf(m, base[(size_t)s * 258 + 256]);
    m = wave_max(m);
    if ((t & 63) == 0) s_red[t >> 6] = m;
    __syncthreads();
    M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    float dsum = 0.0f;
    for (int s = t; s < n_parts; s += 256) {
        const float wgt = expf(base[(size_t)s * 258 + 256] - M);
        s_w[s] = wgt;
        dsum = fmaf(base[(size_t)s * 258 + 257], wgt, dsum);
    }
    dsum = wave_sum(dsum);
    if ((t & 63) == 0) s_red[4 + (t >> 6)] = dsum;
    __syncthreads();
    den = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);
}

__device__ __forceinline__ float lse_num(const float* base, int n_parts, const float* s_w,
                                         float* s_acc, int d0) {
    const int t = threadIdx.x;
    const int d = d0 + (t & 63);
    const int grp = t >> 6;
    // 8 independent chains so the loads of consecutive parts overlap
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int s = grp;
    for (; s + 28 < n_parts; s += 32) {
#pragma unroll
        for (int u = 0; u < 8; u++)
            acc[u] = fmaf(base[(size_t)(s + 4 * u) * 258 + d], s_w[s + 4 * u], acc[u]);
    }
    for (; s < n_parts; s += 4) acc[0] = fmaf(base[(size_t)s * 258 + d], s_w[s], acc[0]);
    const float num = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    s_acc[t] = num;
    __syncthreads();
    return (s_acc[t & 63] + s_acc[64 + (t & 63)]) + (s_acc[128 + (t & 63)] + s_acc[192 + (t & 63)]);
}

__global__ __launch_bounds__(256) void lse_reduce_kernel(const float* __restrict__ part,
                                                        float* __restrict__ out,
                                                        int n_parts) {
    __shared__ float s_w[kMaxParts];
    __shared__ float s_red[8];
    __shared__ float s_acc[256];
    const int qid = blockIdx.x;
    const int d0 = blockIdx.y * 64;
    const float* base = part + (size_t)qid * n_parts * 258;
    float M, den;
    lse_weights(base, n_parts, s_w, s_red, M, den);
    const float num = lse_num(base, n_parts, s_w, s_acc, d0);
    float* o = out + (size_t)qid * 258;
    if (threadIdx.x < 64) o[d0 + threadIdx.x] = num;
    if (blockIdx.y == 0 && threadIdx.x == 0) {
        o[256] = M;
        o[257] = den;
    }
}

// Final merge of all parts of one head + normalise + sigmoid gate -> f16.
__global__ __launch_bounds__(256) void combine_gate_kernel(const float* __restrict__ part,
                                                          const __half* __restrict__ q_gate,
                                                          __half* __restrict__ out,
                                                          int n_parts, float eps) {
    __shared__ float s_w[kMaxParts];
    __shared__ float s_red[8];
    __shared__ float s_acc[256];
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * 64;
    const float* base = part + (size_t)h * n_parts * 258;
    float M, den;
    lse_weights(base, n_parts, s_w, s_red, M, den);
    const float num = lse_num(base, n_parts, s_w, s_acc, d0);
    if (threadIdx.x < 64) {
        const int d = d0 + threadIdx.x;
        float val = num / (den + eps);
        const float g = h2f(q_gate[(size_t)h * 512 + 256 + d]);
        val = val * (1.0f / (1.0f + expf(-g)));
        out[(size_t)h * 256 + d] = __float2half(val);
    }
}

// ref .cu:1983-2010
__global__ void merge_gate_kernel(const float* __restrict__ attn_c,
                                  const float* __restrict__ attn_w,
                                  const __half* __restrict__ q_gate, __half* __restrict__ out,
                                  int H_q, int D, int has_w) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H_q * D) return;
    const int h = i / D, d = i % D;
    const float* cc = attn_c + (size_t)h * (D + 2);
    float num = cc[d], den = cc[D + 1];
    if (has_w) {
        const float* cw = attn_w + (size_t)h * (D + 2);
        const float mc = cc[D], mw = cw[D];
        const float M = fmaxf(mc, mw);
        const float wc = expf(mc - M), ww = expf(mw - M);
        num = fmaf(num, wc, cw[d] * ww);
        den = fmaf(den, wc, cw[D + 1] * ww);
    }
    float val = num / (den + 1e-8f);
    const float g = h2f(q_gate[(size_t)h * 2 * D + D + d]);
    val = val * (1.0f / (1.0f + expf(-g)));
    out[i] = __float2half(val);
}

__global__ void gather_q_kernel(const __half* __restrict__ q_gate, __half* __restrict__ q_out,
                                int H_q, int D) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H_q * D) return;
    q_out[i] = q_gate[(size_t)(i / D) * 2 * D + (i % D)];
}

__global__ void ring_write_kernel(__half* __restrict__ rk, __half* __restrict__ rv,
                                  __half* __restrict__ ru, const __half* __restrict__ k,
                                  const __half* __restrict__ v, const __half* __restrict__ ku,
                                  int kv) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= kv) return;
    if (rk) rk[i] = k[i];
    if (rv) rv[i] = v[i];
    if (ru) ru[i] = ku[i];
}

// ref elementwise_sm75.mojo:1023-1061 (freq = exp(log(theta) * -2i/rot))
__global__ void partial_rope_kernel(__half* __restrict__ vec, int head_dim, int rotary_dim,
                                    int pos, float theta, int stride) {
    const int h = blockIdx.x;
    const int t = threadIdx.x;
    const int half_rot = rotary_dim / 2;
    const int es = stride > 0 ? stride : head_dim;
    for (int i = t; i < half_rot; i += blockDim.x) {
        const float ex = -(float)(2 * i) / (float)rotary_dim;
        const float fr = expf(logf(theta) * ex);
        const float mt = (float)pos * fr;
        const float c = cosf(mt), s = sinf(mt);
        __half* row = vec + (size_t)h * es;
        const float x0 = h2f(row[i]);
        const float x1 = h2f(row[i + half_rot]);
        row[i] = __float2half(fmaf(x0, c, -(x1 * s)));
        row[i + half_rot] = __float2half(fmaf(x0, s, x1 * c));
    }
}

// Front of the attention step of one token (ref:src/models/qwen3_5/
// attention.mojo:329-353) in one launch.  Block b < H_q: query head b of
// q_gate (stride 2 D); block H_q + j: KV head j of k (stride D), whose
// block also copies V head j into the ring.  Per head: RMSNorm over D = 256
// (inv = 1 / sqrt(sum x^2 / D + eps), then (x * inv) * w when a weight is
// given, rounded to fp16 as the reference stores it, elementwise_sm75.mojo:
// 362-423), then half-split RoPE of dims 0..rot-1 at `pos` on the fp16 normed
// values (the partial_rope arithmetic of partial_rope_kernel above).  Outputs:
// q in place; k: normed (pre-RoPE) to ring_u, roped to k in place and to
// ring_k; v to ring_v (ring rows `slot`).
__global__ __launch_bounds__(64) void norm_rope_kernel(NormRopeArgs a) {
    __shared__ float s_x[256];
    const int b = blockIdx.x, t = threadIdx.x;
    const bool is_q = b < a.H_q;
    const int hk = b - a.H_q;
    __half* row = is_q ? a.q_gate + (size_t)b * 512 : a.k + (size_t)hk * 256;
    const float* w = is_q ? a.q_w : a.k_w;
    const uint2 raw = *reinterpret_cast<const uint2*>(row + 4 * t);
    const __half2 p0 = __builtin_bit_cast(__half2, raw.x), p1 = __builtin_bit_cast(__half2, raw.y);
    const float x[4] = {__low2float(p0), __high2float(p0), __low2float(p1), __high2float(p1)};
    float ss = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float inv = (1.0f / sqrtf(ss / 256.0f + a.eps)) * 1.0f;
    __half nh[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float v = x[c] * inv;
        if (w) v *= w[4 * t + c];
        nh[c] = __float2half(v);
        s_x[4 * t + c] = __half2float(nh[c]);
    }
    const size_t slot_off = (size_t)a.slot * a.H_kv * 256 + (size_t)hk * 256 + 4 * t;
    if (!is_q) {
        *reinterpret_cast<uint2*>(a.ring_u + slot_off) =
            uint2{__builtin_bit_cast(uint32_t, __halves2half2(nh[0], nh[1])),
                  __builtin_bit_cast(uint32_t, __halves2half2(nh[2], nh[3]))};
        *reinterpret_cast<uint2*>(a.ring_v + slot_off) =
            *reinterpret_cast<const uint2*>(a.v + (size_t)hk * 256 + 4 * t);
    }
    __syncthreads();
    const int half_rot = a.rot / 2;
    if (t < half_rot) {
        const float ex = -(float)(2 * t) / (float)a.rot;
        const float fr = expf(logf(a.theta) * ex);
        const float mt = (float)a.pos * fr;
        const float c = cosf(mt), s = sinf(mt);
        const float x0 = s_x[t], x1 = s_x[t + half_rot];
        s_x[t] = __half2float(__float2half(fmaf(x0, c, -(x1 * s))));
        s_x[t + half_rot] = __half2float(__float2half(fmaf(x0, s, x1 * c)));
    }
    __syncthreads();
    const uint2 outw = uint2{__builtin_bit_cast(uint32_t, __floats2half2_rn(s_x[4 * t], s_x[4 * t + 1])),
                             __builtin_bit_cast(uint32_t, __floats2half2_rn(s_x[4 * t + 2], s_x[4 * t + 3]))};
    *reinterpret_cast<uint2*>(row + 4 * t) = outw;
    if (!is_q) *reinterpret_cast<uint2*>(a.ring_k + slot_off) = outw;
}

// ------------------------------------------------------------ dispatchers
hipError_t launch_attn_parts(const AttnArgs& a, int n_rep, dim3 grid, hipStream_t st) {
    switch (n_rep) {
#define KHQ_CASE(N) \
    case N: hipLaunchKernelGGL(attn_part_kernel<N>, grid, dim3(256), 0, st, a); break;
        KHQ_CASE(1) KHQ_CASE(2) KHQ_CASE(3) KHQ_CASE(4)
        KHQ_CASE(5) KHQ_CASE(6) KHQ_CASE(7) KHQ_CASE(8)
#undef KHQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_window_parts(const WinArgs& a, int n_rep, dim3 grid, hipStream_t st) {
    switch (n_rep) {
#define KHQ_CASE(N) \
    case N: hipLaunchKernelGGL(window_part_kernel<N>, grid, dim3(256), 0, st, a); break;
        KHQ_CASE(1) KHQ_CASE(2) KHQ_CASE(3) KHQ_CASE(4)
        KHQ_CASE(5) KHQ_CASE(6) KHQ_CASE(7) KHQ_CASE(8)
#undef KHQ_CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_compress(const __half* x, const __half* d_vec, const __half* rotor,
                           const __half* cents, const __half* vq, uint32_t* out_mask,
                           __half* out_norms, __half* out_rn, uint8_t* out_pay,
                           uint8_t* out_sm, int n, float ts, float alpha, int is_v,
                           hipStream_t st) {
    const int blocks = is_v ? n : (n + 3) / 4;
    hipLaunchKernelGGL(compress_kernel, dim3(blocks), dim3(256), 0, st, x, d_vec, rotor, cents,
                       vq, out_mask, out_norms, out_rn, out_pay, out_sm, n, ts, alpha, is_v);
    return hipGetLastError();
}

hipError_t launch_compress_pair(const CompressJob& k, const CompressJob& v, hipStream_t st) {
    const int nb_k = (k.n + 3) / 4;
    hipLaunchKernelGGL(compress_pair_kernel, dim3(nb_k + v.n), dim3(256), 0, st, k, v, nb_k);
    return hipGetLastError();
}

hipError_t launch_lse_reduce(const float* part, float* out, int n_q, int n_parts,
                             hipStream_t st) {
    if (n_parts > kMaxParts) return hipErrorInvalidValue;
    hipLaunchKernelGGL(lse_reduce_kernel, dim3(n_q, 4), dim3(256), 0, st, part, out, n_parts);
    return hipGetLastError();
}

hipError_t launch_combine_gate(const float* part, const __half* q_gate, __half* out, int H_q,
                               int n_parts, float eps, hipStream_t st) {
    if (n_parts > kMaxParts) return hipErrorInvalidValue;
    hipLaunchKernelGGL(combine_gate_kernel, dim3(H_q, 4), dim3(256), 0, st, part, q_gate, out,
                       n_parts, eps);
    return hipGetLastError();
}

hipError_t launch_merge_gate(const float* ac, const float* aw, const __half* qg, __half* out,
                             int H_q, int D, int has_w, hipStream_t st) {
    const int total = H_q * D;
    hipLaunchKernelGGL(merge_gate_kernel, dim3((total + 255) / 256), dim3(256), 0, st, ac, aw,
                       qg, out, H_q, D, has_w);
    return hipGetLastError();
}

hipError_t launch_gather_q(const __half* qg, __half* qo, int H_q, int D, hipStream_t st) {
    const int total = H_q * D;
    hipLaunchKernelGGL(gather_q_kernel, dim3((total + 255) / 256), dim3(256), 0, st, qg, qo,
                       H_q, D);
    return hipGetLastError();
}

hipError_t launch_ring_write(__half* rk, __half* rv, __half* ru, const __half* k,
                             const __half* v, const __half* ku, int kv, hipStream_t st) {
    hipLaunchKernelGGL(ring_write_kernel, dim3((kv + 255) / 256), dim3(256), 0, st, rk, rv, ru,
                       k, v, ku, kv);
    return hipGetLastError();
}

hipError_t launch_partial_rope(__half* vec, int num_heads, int head_dim, int rotary_dim, int pos,
                               float theta, int stride, hipStream_t st) {
    hipLaunchKernelGGL(partial_rope_kernel, dim3(num_heads), dim3(64), 0, st, vec, head_dim,
                       rotary_dim, pos, theta, stride);
    return hipGetLastError();
}

hipError_t launch_norm_rope(const NormRopeArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(norm_rope_kernel, dim3(a.H_q + a.H_kv), dim3(64), 0, st, a);
    return hipGetLastError();
}

}  // namespace khq
