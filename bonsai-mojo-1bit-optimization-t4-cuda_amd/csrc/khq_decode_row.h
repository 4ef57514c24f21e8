// khq_decode_row.h -- decode of one compressed (token, KV head) row by one
// wavefront, lane p owning patch p (dims 4 p .. 4 p + 3): the K row with its
// RoPE (dims 0..63) and the V row, both to fp32 in the head's natural basis.
// Shared by the decode launch (fields read from the payload arrays) and the
// compression launch that decodes the rows it has just packed (fields taken
// from its LDS staging), so the two produce the same bits.
// Format and steps: the compressed-region attention kernel's per-row decode,
// ref src/csrc/qmv_sm75_kernel.cu:1608-1699 (K) and :1739-1762 (V); the RoPE
// is the partial rotary of attention.mojo:348-353.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "khq_internal.h"
#include "khq_mfma_util.h"

namespace khq {
namespace dec {

// Per-lane constants of a layer (centroids, rotors, 1 / d scales, RoPE
// frequencies of the lane's dims).
struct Consts {
    float cbk[4], ldk[4], ldv[4], rk[16], rv[16], fr[4];
    float cv0, cv1;
    uint64_t below;  // lanes below p
};

__device__ __forceinline__ void load_consts(const DecompArgs& a, int p, Consts& c) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        c.cbk[i] = __half2float(a.cents_k[512 + 4 * p + i]);
        c.ldk[i] = (1.0f / 256.0f) / (__half2float(a.dk[4 * p + i]) + 1e-8f);
        c.ldv[i] = (1.0f / 16.0f) / (__half2float(a.dv[4 * p + i]) + 1e-8f);
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        c.rk[i] = __half2float(a.rotor_k[p * 16 + i]);
        c.rv[i] = __half2float(a.rotor_v[p * 16 + i]);
    }
    c.cv0 = __half2float(a.cents_v[4 * p + 3]) * a.a_v;
    c.cv1 = __half2float(a.cents_v[256 + 4 * p + 3]) * a.a_v;
    // RoPE frequencies of dims 4 (p & 7) + i (lanes 0..15 rotate dims 0..63)
#pragma unroll
    for (int i = 0; i < 4; i++) c.fr[i] = powf(a.rope_base, -2.0f * (float)(4 * (p & 7) + i) / 64.0f);
    c.below = (p == 0) ? 0ull : (~0ull >> (64 - p));
}

__device__ __forceinline__ uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// K row: mw = mask word p >> 2 (codes of the lane's 4 dims at bits
// 2 (4 (p & 3) + k)), kb = the 40 payload bytes, nk / rs = the row's fp16 norm
// and residual scale as floats, pos = the token's absolute position.
__device__ __forceinline__ void decode_k(const DecompArgs& a, const Consts& c, uint32_t mw,
                                         const uint8_t* kb, float nk, float rs, float pos, int p,
                                         float (&y)[4]) {
    float mult = (float)rd32(kb) / 1000.0f;
    if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
    uint32_t code[4];
    int own = 0, ord = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        code[k] = (mw >> (2 * (4 * (p & 3) + k))) & 3u;
        const uint64_t b = __ballot(code[k] == 3u);
        ord += __popcll(b & c.below);
    }
    float kf[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float cbase = c.cbk[k] * mult;
        float kv = 0.0f;
        if (code[k] == 3u) {
            const int jo = ord + own;
            const float sign = (jo < 50 && ((kb[29 + jo / 8] >> (jo % 8)) & 1)) ? 1.0f : -1.0f;
            const float r4 = (jo < 50) ? (float)((kb[4 + jo / 2] >> ((jo % 2) * 4)) & 0xF) : 0.0f;
            kv = sign * fmaf(r4, rs, cbase);
            own++;
        } else if (code[k] == 2u) {
            kv = cbase;
        } else if (code[k] == 1u) {
            kv = -cbase;
        }
        kf[k] = kv * a.a_k * nk;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float s = kf[0] * c.rk[i * 4 + 0];
        s = fmaf(kf[1], c.rk[i * 4 + 1], s);
        s = fmaf(kf[2], c.rk[i * 4 + 2], s);
        s = fmaf(kf[3], c.rk[i * 4 + 3], s);
        y[i] = s;
    }
    mu::fwht256(y, p);
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] *= c.ldk[i];
    // RoPE on dims 0..63: lane p < 8 holds dim i, lane p + 8 dim i + 32
    float xo[4];
#pragma unroll
    for (int i = 0; i < 4; i++) xo[i] = __shfl_xor(y[i], 8, 64);
    if (p < 16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float cs, sn;
            mu::sincos_rev(pos * c.fr[i], cs, sn);
            y[i] = p < 8 ? fmaf(y[i], cs, -(xo[i] * sn)) : fmaf(xo[i], sn, y[i] * cs);
        }
    }
}

// V row: vc (decode_v) = the patch's 8-bit codebook index, pvl = its 12-bit field
// (bit 7 the dim-3 centroid, bits 8..11 the dim-3 residual), nv / ec / smv =
// the row's fp16 norm, fp16 energy ratio (as floats) and fp32 shared meta.
// y = the decoded dims, 1 / (16 d_v) applied.
// cbv = the patch's codebook entry (three fp16 values as floats).
__device__ __forceinline__ void decode_v_cb(const DecompArgs& a, const Consts& c, const float (&cbv)[3],
                                            uint32_t pvl, float nv, float ec, float smv, int p,
                                            float (&y)[4]) {
    const float pre_v = (a.a_v * nv) * ec;
    const float pre_r = smv * nv;
    float vv[4];
#pragma unroll
    for (int k = 0; k < 3; k++) vv[k] = cbv[k] * pre_v;
    vv[3] = fmaf(((float)((pvl >> 8) & 0xFu) - 8.0f) / 7.0f, pre_r,
                 (((pvl >> 7) & 1u) ? c.cv1 : c.cv0) * nv);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float s = vv[0] * c.rv[i * 4 + 0];
        s = fmaf(vv[1], c.rv[i * 4 + 1], s);
        s = fmaf(vv[2], c.rv[i * 4 + 2], s);
        s = fmaf(vv[3], c.rv[i * 4 + 3], s);
        y[i] = s;
    }
    mu::fwht256(y, p);
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] *= c.ldv[i];
}

__device__ __forceinline__ void decode_v(const DecompArgs& a, const Consts& c, uint32_t vc,
                                         uint32_t pvl, float nv, float ec, float smv, int p,
                                         float (&y)[4]) {
    float cbv[3];
#pragma unroll
    for (int k = 0; k < 3; k++) cbv[k] = __half2float(a.vq[(size_t)p * 768 + vc * 3 + k]);
    decode_v_cb(a, c, cbv, pvl, nv, ec, smv, p, y);
}

}  // namespace dec
}  // namespace khq
