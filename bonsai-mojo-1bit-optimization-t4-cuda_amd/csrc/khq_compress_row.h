// khq_compress_row.h -- the compression of one 256-dim row into the KHQ
// packed format (ref src/csrc/qmv_sm75_kernel.cu:1256-1467), one wavefront
// per K row and one block per V row, and the lane-per-patch helpers it uses.
// Included by the compression launches (khq_kernels.hip) and by the launch
// that compresses a chunk, decodes it back into the dense key space and
// appends the new tokens in one grid (khq_prefill.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "khq_internal.h"
#include "khq_decode_row.h"

namespace khq {

__device__ __forceinline__ float h2f(__half h) { return __half2float(h); }

__device__ __forceinline__ uint64_t lanemask_lt() {
    const unsigned lane = threadIdx.x & 63u;
    return lane == 0 ? 0ull : (~0ull >> (64u - lane));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Butterfly across lanes: lower lane (bit m clear) keeps a+b, upper keeps a-b
// where a is the lower lane's value.  Same operands and order as the
// in-place FWHT of the reference (a + b, a - b).
__device__ __forceinline__ float xbfly(float x, int m, bool lower) {
    float p = __shfl_xor(x, m, 64);
    return lower ? (x + p) : (p - x);
}

// FWHT-256 on a wavefront holding 4 consecutive dims per lane.
__device__ __forceinline__ void fwht256(float (&v)[4]) {
    const int lane = threadIdx.x & 63;
    float a = v[0], b = v[1];
    v[0] = a + b; v[1] = a - b;
    a = v[2]; b = v[3];
    v[2] = a + b; v[3] = a - b;
    a = v[0]; b = v[2];
    v[0] = a + b; v[2] = a - b;
    a = v[1]; b = v[3];
    v[1] = a + b; v[3] = a - b;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const bool lower = (lane & m) == 0;
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = xbfly(v[c], m, lower);
    }
}

// Sequential folds of LDS rows in index order (the reference's order), the
// reads issued a batch at a time ahead of the batch's dependent chain (one
// LDS round trip per batch instead of per element).
__device__ __forceinline__ float fold_sq256(const float* v) {
    float s = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < 256; i0 += 32) {
        float4 t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) t[j] = *reinterpret_cast<const float4*>(&v[i0 + 4 * j]);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            s = fmaf(t[j].x, t[j].x, s);
            s = fmaf(t[j].y, t[j].y, s);
            s = fmaf(t[j].z, t[j].z, s);
            s = fmaf(t[j].w, t[j].w, s);
        }
    }
    return s;
}
// sa = a[0] + a[1] + ..., sb likewise, over n (a multiple of 16) elements
__device__ __forceinline__ void fold_sum2(const float* a, const float* b, int n, float& sa,
                                          float& sb) {
    sa = 0.0f;
    sb = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < n; i0 += 16) {
        float4 ta[4], tb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ta[j] = *reinterpret_cast<const float4*>(&a[i0 + 4 * j]);
            tb[j] = *reinterpret_cast<const float4*>(&b[i0 + 4 * j]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sa += ta[j].x; sa += ta[j].y; sa += ta[j].z; sa += ta[j].w;
            sb += tb[j].x; sb += tb[j].y; sb += tb[j].z; sb += tb[j].w;
        }
    }
}

// ---------------------------------------------------------------- compress
// One wavefront per row, four rows per 256-thread block.  The reference
// (ref:src/csrc/qmv_sm75_kernel.cu:1256-1467) runs one thread per row; the
// three order-sensitive sums (sum of squares, sum_normals/sum_cbase, the V
// energies) are kept sequential here by staging the terms in LDS and letting
// every lane fold them in index order.
//
// DEC: the rows are also decoded back into the dense key space (roped K row
// at key key0 + token, V^T column key0 + token of da), from the fields just
// packed, rounded as they are stored, so the result is the decode launch's.
// Row r of the job is (token r / h_kv, KV head r % h_kv) of da.
template <bool DEC = false>
__device__ __forceinline__ void compress_block(
    const __half* __restrict__ x, const __half* __restrict__ d_vec,
    const __half* __restrict__ rotor, const __half* __restrict__ cents,
    const __half* __restrict__ vq, uint32_t* __restrict__ out_mask,
    __half* __restrict__ out_norms, __half* __restrict__ out_rn,
    uint8_t* __restrict__ out_pay, uint8_t* __restrict__ out_sm, int n, float ts,
    float alpha, int is_v, int bid, const DecompArgs* da = nullptr) {
    __shared__ float s_a[4][256];
    __shared__ float s_b[4][256];
    __shared__ uint32_t s_w[4][32];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    // K: one row per wavefront.  V: one row per block, the four wavefronts
    // search a quarter of the codebook each and all finish the row; wavefront
    // 0 writes it.
    const int row = is_v ? bid : bid * 4 + wave;
    const bool valid = row < n;
    const bool live = valid && (!is_v || wave == 0);
    const float f_s = 0.0625f;
    dec::Consts dcs;
    if constexpr (DEC) dec::load_consts(*da, lane, dcs);
    // every per-lane constant is requested here, so the block waits for
    // memory once instead of once per phase
    float dv4[4], rot[16], cbk[4];
#pragma unroll
    for (int c = 0; c < 4; c++) dv4[c] = h2f(d_vec[lane * 4 + c]);
#pragma unroll
    for (int i = 0; i < 16; i++) rot[i] = h2f(rotor[lane * 16 + i]);
    // K: the code-1/2 centroid of the lane's dims; V: the dim-3 centroids
#pragma unroll
    for (int c = 0; c < 4; c++)
        cbk[c] = is_v ? h2f(cents[(c & 1) * 256 + lane * 4 + 3]) : h2f(cents[2 * 256 + lane * 4 + c]);

    // A V row's four wavefronts share one row: wavefront 0 computes its
    // projection and hands it to the others through LDS (the search below
    // is what needs all four).
    __shared__ float s_pj[256];
    const bool own_row = !is_v || wave == 0;  // uniform per wavefront
    float xv[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid && own_row) {
        const __half* xr = x + (size_t)row * 256 + lane * 4;
#pragma unroll
        for (int c = 0; c < 4; c++) xv[c] = h2f(xr[c]);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) s_a[wave][lane * 4 + c] = xv[c];
    if (lane < 32) s_w[wave][lane] = 0u;
    __syncthreads();
    float norm = 0.0f;
    float proj[4] = {0.f, 0.f, 0.f, 0.f};
    if (own_row) {
        const float sum_sq = fold_sq256(s_a[wave]);
        norm = sqrtf(sum_sq + 1e-8f);
        if (live && lane == 0) out_norms[row] = __float2half(norm);

        float r[4];
#pragma unroll
        for (int c = 0; c < 4; c++) r[c] = (xv[c] * dv4[c]) / (norm + 1e-8f);
        fwht256(r);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float acc = r[0] * rot[0 * 4 + c];
            acc = fmaf(r[1], rot[1 * 4 + c], acc);
            acc = fmaf(r[2], rot[2 * 4 + c], acc);
            acc = fmaf(r[3], rot[3 * 4 + c], acc);
            proj[c] = acc * f_s;
        }
        if (is_v) {
#pragma unroll
            for (int c = 0; c < 4; c++) s_pj[lane * 4 + c] = proj[c];
        }
    }
    __syncthreads();  // s_a reused below; a V row's projection in place
    if (is_v && wave != 0) {
#pragma unroll
        for (int c = 0; c < 4; c++) proj[c] = s_pj[lane * 4 + c];
    }

    if (!is_v) {
        // ---- K branch, ref .cu:1314-1351 and :1429-1466
        bool cand[4];
#pragma unroll
        for (int c = 0; c < 4; c++) cand[c] = fabsf(proj[c]) > 1.60f * f_s;
        const uint64_t lt = lanemask_lt();
        unsigned base = 0, total = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint64_t b = __ballot(cand[c]);
            base += (unsigned)__popcll(b & lt);
            total += (unsigned)__popcll(b);
        }
        const unsigned n_out = total < 50u ? total : 50u;
        unsigned code[4], ord[4];
        unsigned run = base;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            ord[c] = run;
            float sa = 0.0f, sb = 0.0f;
            if (cand[c]) {
                code[c] = (run < 50u) ? 3u : (proj[c] > 0.0f ? 2u : 1u);
                run++;
            } else {
                code[c] = proj[c] > 0.47f * f_s ? 2u : (proj[c] < -0.47f * f_s ? 1u : 0u);
                if (code[c] != 0u) {
                    sa = fabsf(proj[c]);
                    sb = cbk[c];
                }
            }
            s_a[wave][lane * 4 + c] = sa;
            s_b[wave][lane * 4 + c] = sb;
        }
        unsigned byte = code[0] | (code[1] << 2) | (code[2] << 4) | (code[3] << 6);
        atomicOr(&s_w[wave][16 + (lane >> 2)], byte << (8 * (lane & 3)));
        __syncthreads();
        float sum_normals, sum_cbase;
        fold_sum2(s_a[wave], s_b[wave], 256, sum_normals, sum_cbase);
        float mult = (sum_cbase > 1e-5f) ? (sum_normals / sum_cbase) : 1.0f;
        if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
        float res[4] = {0.f, 0.f, 0.f, 0.f};
        float my_max = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if (code[c] == 3u) {
                const float cb = cbk[c];
                res[c] = fmaxf(0.0f, fmaf(-cb, mult, fabsf(proj[c] * ts)));
                my_max = fmaxf(my_max, res[c]);
            }
        }
        const float max_res = wave_max(my_max);
        const float rs = (n_out > 0u) ? (fmaxf(max_res, 1e-4f) / 15.0f) : 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if (code[c] == 3u) {
                const unsigned j = ord[c];
                if (rs > 0.0f) {
                    const float r4 = roundf(res[c] / rs);
                    const unsigned rv = (unsigned)(uint8_t)fmaxf(0.0f, fminf(15.0f, r4));
                    const unsigned by = 4u + j / 2u;
                    atomicOr(&s_w[wave][by >> 2], rv << (8u * (by & 3u) + 4u * (j & 1u)));
                }
                if (proj[c] > 0.0f) {
                    const unsigned by = 29u + j / 8u;
                    atomicOr(&s_w[wave][by >> 2], 1u << (8u * (by & 3u) + (j & 7u)));
                }
            }
        }
        if (lane == 0) {
            atomicOr(&s_w[wave][0], (unsigned)(mult * 1000.0f));
            atomicOr(&s_w[wave][9], 0x02u);
        }
        __syncthreads();
        if (live) {
            if (lane < 16) out_mask[(size_t)row * 16 + lane] = s_w[wave][16 + lane];
            if (lane < 10)
                reinterpret_cast<uint32_t*>(out_pay + (size_t)row * 40)[lane] = s_w[wave][lane];
            if (lane == 0) {
                out_rn[row] = __float2half(rs);
                if (out_sm) *reinterpret_cast<uint32_t*>(out_sm + (size_t)row * 4) = 0u;
            }
        }
        if constexpr (DEC) {
            if (valid) {  // uniform per wavefront
                const int tok = row / da->h_kv, h = row - tok * da->h_kv;
                float y[4];
                dec::decode_k(*da, dcs, s_w[wave][16 + (lane >> 2)],
                              reinterpret_cast<const uint8_t*>(s_w[wave]),
                              h2f(__float2half(norm)), h2f(__float2half(rs)),
                              (float)(da->start_pos + da->tok0 + tok), lane, y);
                *reinterpret_cast<uint2*>(da->out_k +
                                          ((size_t)(da->key0 + tok) * da->h_kv + h) * 256 + 4 * lane) =
                    uint2{mu::pk_rne(y[0], y[1]), mu::pk_rne(y[2], y[3])};
            }
        }
        return;
    }

    // ---- V branch, ref .cu:1353-1428: lane p owns patch p
    const float v0 = proj[0], v1 = proj[1], v2 = proj[2], v3 = proj[3];
    float best_d = 1e20f;
    unsigned best = 0;
    // the lane's codebook quarter (codes 64 wave .. + 63) in two chunks of 32
    // codes (12 x 16 B), the second chunk's loads in flight while the first
    // is searched; codes in increasing order with a strict < (first minimum
    // wins), then the quarters in order through LDS, so the result is the
    // sequential search's
    const uint4* cb4 = reinterpret_cast<const uint4*>(vq + (size_t)lane * 768);
    uint4 cur[12], nxt[12];
#pragma unroll
    for (int k = 0; k < 12; k++) cur[k] = cb4[12 * (2 * wave) + k];
    for (int ch = 2 * wave; ch < 2 * wave + 2; ch++) {
        if (ch + 1 < 2 * wave + 2) {
#pragma unroll
            for (int k = 0; k < 12; k++) nxt[k] = cb4[12 * (ch + 1) + k];
        }
        const uint16_t* hv = reinterpret_cast<const uint16_t*>(cur);
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float d0 = fmaf(-h2f(__ushort_as_half(hv[3 * j + 0])), alpha, v0);
            const float d1 = fmaf(-h2f(__ushort_as_half(hv[3 * j + 1])), alpha, v1);
            const float d2 = fmaf(-h2f(__ushort_as_half(hv[3 * j + 2])), alpha, v2);
            const float dist = fmaf(d2, d2, fmaf(d1, d1, d0 * d0));
            if (dist < best_d) { best_d = dist; best = 32u * ch + j; }
        }
#pragma unroll
        for (int k = 0; k < 12; k++) cur[k] = nxt[k];
    }
    {
        __shared__ float s_bd[4][64];
        __shared__ unsigned s_bi[4][64];
        s_bd[wave][lane] = best_d;
        s_bi[wave][lane] = best;
        __syncthreads();
        best_d = s_bd[0][lane];
        best = s_bi[0][lane];
#pragma unroll
        for (int w = 1; w < 4; w++)
            if (s_bd[w][lane] < best_d) {
                best_d = s_bd[w][lane];
                best = s_bi[w][lane];
            }
    }
    const __half* cbp = vq + (size_t)lane * 768;
    const float cbh[3] = {h2f(cbp[best * 3]), h2f(cbp[best * 3 + 1]), h2f(cbp[best * 3 + 2])};
    const float c0 = cbh[0] * alpha;
    const float c1 = cbh[1] * alpha;
    const float c2 = cbh[2] * alpha;
    const float te = fmaf(v2, v2, fmaf(v1, v1, v0 * v0));
    const float ve = fmaf(c2, c2, fmaf(c1, c1, c0 * c0));
    const float cv0 = cbk[0];
    const float cv1 = cbk[1];
    const float dd0 = fabsf(fmaf(-cv0, alpha, v3));
    const float dd1 = fabsf(fmaf(-cv1, alpha, v3));
    unsigned bs = 0;
    float best_s = 1e20f;
    if (dd0 < best_s) { best_s = dd0; bs = 0; }
    if (dd1 < best_s) { best_s = dd1; bs = 1; }
    const float resid = fmaf(-(bs ? cv1 : cv0), alpha, v3);
    const float max_res = wave_max(fabsf(resid));
    const float res_scale = fmaxf(max_res, 1e-4f);
    const float scaled = fmaf(resid / res_scale, 7.0f, 8.0f);
    const unsigned dump = (unsigned)fmaxf(0.0f, fminf(15.0f, roundf(scaled)));
    const unsigned pv = (best & 0x7Fu) | ((bs & 1u) << 7) | ((dump & 0xFu) << 8);
    const uint64_t hi = __ballot(((best >> 7) & 1u) != 0u);
    s_a[wave][lane] = te;
    s_b[wave][lane] = ve;
    __shared__ uint32_t s_pv[4][64];
    s_pv[wave][lane] = pv;
    __syncthreads();
    if (!live) return;
    uint32_t* op = reinterpret_cast<uint32_t*>(out_pay + (size_t)row * 104);
    if (lane < 8) {
        const uint32_t* p = &s_pv[wave][lane * 8];
        op[lane * 3 + 0] = p[0] | (p[1] << 12) | ((p[2] & 0xFFu) << 24);
        op[lane * 3 + 1] = (p[2] >> 8) | (p[3] << 4) | (p[4] << 16) | ((p[5] & 0xFu) << 28);
        op[lane * 3 + 2] = (p[5] >> 4) | (p[6] << 8) | (p[7] << 20);
    } else if (lane == 8) {
        op[24] = (uint32_t)(hi & 0xFFFFFFFFull);
        op[25] = (uint32_t)(hi >> 32);
    } else if (lane == 9) {
        float st, sv;
        fold_sum2(s_a[wave], s_b[wave], 64, st, sv);
        out_rn[row] = __float2half(sqrtf(st / (sv + 1e-8f)));
        *reinterpret_cast<float*>(out_sm + (size_t)row * 4) = max_res;
    }
    if constexpr (DEC) {
        // the energy ratio as lane 9 folds it, on every lane
        float st, sv;
        fold_sum2(s_a[wave], s_b[wave], 64, st, sv);
        const float ec = h2f(__float2half(sqrtf(st / (sv + 1e-8f))));
        const int tok = row / da->h_kv, h = row - tok * da->h_kv;
        float y[4];
        dec::decode_v_cb(*da, dcs, cbh, pv, h2f(__float2half(norm)), ec, max_res, lane, y);
        _Float16* vt = reinterpret_cast<_Float16*>(da->out_vt);
#pragma unroll
        for (int c = 0; c < 4; c++)
            vt[((size_t)h * 256 + 4 * lane + c) * da->ld_vt + da->key0 + tok] = (_Float16)y[c];
    }
}

}  // namespace khq
