/*
 * khq_oracle.c -- CPU restatement of the KHQ decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library and the CPU baseline timed by bench.py; nothing in the product path
 * links or calls it.  It is built by oracle/Makefile into oracle/libkhq_oracle.so.
 *
 * Every function restates one reference kernel or host routine of
 * oki-abrian/bonsai-mojo-1bit-optimization-t4-cuda (file:line cited per
 * function).  The reference is CUDA compiled by nvcc with -fmad=true, whose
 * exact contraction choices cannot be observed here.  This oracle fixes them
 * explicitly with fmaf() where nvcc would contract a multiply feeding an add
 * (built with -ffp-contract=off so the compiler adds none of its own).  The
 * HIP compress kernel uses the very same operation sequence, which is what
 * makes packed codes bit-exact between the two; attention outputs are judged
 * by tolerance.
 *
 * fp16 <-> fp32 conversion is round-to-nearest-even, as __float2half.
 * f_s = rsqrtf(256) is taken as exactly 0.0625.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define KHQ_D 256
#define KHQ_NP 64
#define KHQ_MAX_OUTLIERS 50

/* ------------------------------------------------------------------ fp16 */
float khq_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400) == 0);
            man &= 0x3FF;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t khq_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00 | (absx > 0x7F800000u ? 0x200 : 0));
    }
    if (absx >= 0x477FF000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00);
    }
    if (absx < 0x38800000u) { /* below fp16 normal range: subnormal or 0 */
        if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7FFFFF) | 0x800000;
        /* value = m * 2^(e-150); in units of 2^-24 that is m >> (126 - e),
         * with the shift in [14, 24] here, rounded to nearest even */
        uint32_t sh = 126u - e;
        uint32_t q = m >> sh;
        uint32_t rem = m & ((1u << sh) - 1);
        uint32_t half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112;
    uint32_t m = absx & 0x7FFFFF;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

void khq_f2h_array(const float* in, uint16_t* out, long n) {
    for (long i = 0; i < n; i++) out[i] = khq_f2h(in[i]);
}

void khq_h2f_array(const uint16_t* in, float* out, long n) {
    for (long i = 0; i < n; i++) out[i] = khq_h2f(in[i]);
}

static inline uint32_t rd_u32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}
static inline void wr_u32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }
static inline float rd_f32(const uint8_t* p) {
    float v;
    memcpy(&v, p, 4);
    return v;
}
static inline void wr_f32(uint8_t* p, float v) { memcpy(p, &v, 4); }

/* ------------------------------------------------------------- compress */
/* Restates khq_compress_kernel, ref:src/csrc/qmv_sm75_kernel.cu:1256-1467,
 * one row at a time (the reference runs one thread per row). */
static void compress_row(const uint16_t* xrow, const uint16_t* d_vec,
                         const uint16_t* rotor, const uint16_t* cents,
                         const uint16_t* vq, uint32_t* out_mask_row,
                         uint16_t* out_norm, uint16_t* out_rn,
                         uint8_t* pay, uint8_t* smeta, float ts, float alpha,
                         int is_v) {
    const float f_s = 0.0625f;
    /* .cu:1274-1280 sequential sum of squares */
    float sum_sq = 0.0f;
    for (int i = 0; i < KHQ_D; i++) {
        float v = khq_h2f(xrow[i]);
        sum_sq = fmaf(v, v, sum_sq);
    }
    float norm = sqrtf(sum_sq + 1e-8f);
    *out_norm = khq_f2h(norm);

    /* .cu:1282-1292 normalise with d, in-place unnormalised FWHT-256 */
    float r[KHQ_D];
    for (int i = 0; i < KHQ_D; i++)
        r[i] = (khq_h2f(xrow[i]) * khq_h2f(d_vec[i])) / (norm + 1e-8f);
    for (int step = 1; step < KHQ_D; step <<= 1)
        for (int i = 0; i < KHQ_D; i += 2 * step)
            for (int j = 0; j < step; j++) {
                float a = r[i + j], b = r[i + j + step];
                r[i + j] = a + b;
                r[i + j + step] = a - b;
            }

    /* .cu:1294-1303 per-patch rotor: rot[c] = sum_k r[k] * R[k*4+c] */
    float rot[KHQ_D];
    for (int p = 0; p < KHQ_NP; p++)
        for (int c = 0; c < 4; c++) {
            const uint16_t* R = rotor + p * 16;
            float acc = r[p * 4 + 0] * khq_h2f(R[0 * 4 + c]);
            acc = fmaf(r[p * 4 + 1], khq_h2f(R[1 * 4 + c]), acc);
            acc = fmaf(r[p * 4 + 2], khq_h2f(R[2 * 4 + c]), acc);
            acc = fmaf(r[p * 4 + 3], khq_h2f(R[3 * 4 + c]), acc);
            rot[p * 4 + c] = acc;
        }

    if (!is_v) {
        /* .cu:1314-1351 K codes */
        uint32_t plan[16] = {0};
        float o_abs[KHQ_MAX_OUTLIERS];
        uint32_t o_dim[KHQ_MAX_OUTLIERS];
        uint32_t o_sign[KHQ_MAX_OUTLIERS];
        uint32_t n_out = 0;
        float sum_normals = 0.0f, sum_cbase = 0.0f;
        for (int i = 0; i < KHQ_D; i++) {
            float proj = rot[i] * f_s;
            float proj_scaled = proj * ts;
            float abs_proj = fabsf(proj);
            uint32_t code;
            if (abs_proj > 1.60f * f_s) {
                if (n_out < KHQ_MAX_OUTLIERS) {
                    code = 3;
                    o_abs[n_out] = fabsf(proj_scaled);
                    o_dim[n_out] = (uint32_t)i;
                    o_sign[n_out] = proj > 0.0f ? 1u : 0u;
                    n_out++;
                } else {
                    code = proj > 0.0f ? 2u : 1u;
                }
            } else {
                if (proj > 0.47f * f_s) code = 2;
                else if (proj < -0.47f * f_s) code = 1;
                else code = 0;
                if (code == 1 || code == 2) {
                    sum_normals += abs_proj;
                    sum_cbase += khq_h2f(cents[2 * KHQ_D + i]);
                }
            }
            plan[i / 16] |= code << ((i % 16) * 2);
        }
        for (int k = 0; k < 16; k++) out_mask_row[k] = plan[k];
        /* .cu:1429-1466 multiplier, residuals, packing */
        float mult = (sum_cbase > 1e-5f) ? (sum_normals / sum_cbase) : 1.0f;
        if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
        float max_res = 0.0f;
        float res[KHQ_MAX_OUTLIERS];
        for (uint32_t j = 0; j < n_out; j++) {
            float cb = khq_h2f(cents[2 * KHQ_D + o_dim[j]]);
            float rj = fmaxf(0.0f, fmaf(-cb, mult, o_abs[j]));
            res[j] = rj;
            if (rj > max_res) max_res = rj;
        }
        float rs = (n_out > 0) ? (fmaxf(max_res, 1e-4f) / 15.0f) : 0.0f;
        *out_rn = khq_f2h(rs);
        memset(pay, 0, 40);
        wr_u32(pay, (uint32_t)(mult * 1000.0f));
        for (uint32_t j = 0; j < n_out; j++) {
            if (rs > 0.0f) {
                float r4 = roundf(res[j] / rs);
                uint8_t rv = (uint8_t)fmaxf(0.0f, fminf(15.0f, r4));
                pay[4 + j / 2] |= (uint8_t)(rv << ((j % 2) * 4));
            }
        }
        for (uint32_t j = 0; j < n_out; j++)
            if (o_sign[j]) pay[29 + j / 8] |= (uint8_t)(1u << (j % 8));
        pay[36] = 0x02;
        wr_u32(smeta, 0u);
        return;
    }

    /* .cu:1353-1428 V branch: VQ on dims 0..2, binary centroid on dim 3 */
    uint32_t vq_code[KHQ_NP], d3_code[KHQ_NP], d3_dump[KHQ_NP];
    float pres[KHQ_NP], te[KHQ_NP], ve[KHQ_NP];
    float max_res = 0.0f;
    for (int p = 0; p < KHQ_NP; p++) {
        float v0 = rot[p * 4 + 0] * f_s;
        float v1 = rot[p * 4 + 1] * f_s;
        float v2 = rot[p * 4 + 2] * f_s;
        const uint16_t* cb = vq + p * 256 * 3;
        float best_d = 1e20f;
        uint32_t best = 0;
        for (uint32_t i = 0; i < 256; i++) {
            float d0 = fmaf(-khq_h2f(cb[i * 3 + 0]), alpha, v0);
            float d1 = fmaf(-khq_h2f(cb[i * 3 + 1]), alpha, v1);
            float d2 = fmaf(-khq_h2f(cb[i * 3 + 2]), alpha, v2);
            float dist = fmaf(d2, d2, fmaf(d1, d1, d0 * d0));
            if (dist < best_d) { best_d = dist; best = i; }
        }
        vq_code[p] = best;
        float c0 = khq_h2f(cb[best * 3 + 0]) * alpha;
        float c1 = khq_h2f(cb[best * 3 + 1]) * alpha;
        float c2 = khq_h2f(cb[best * 3 + 2]) * alpha;
        te[p] = fmaf(v2, v2, fmaf(v1, v1, v0 * v0));
        ve[p] = fmaf(c2, c2, fmaf(c1, c1, c0 * c0));
        float v3 = rot[p * 4 + 3] * f_s;
        float best_s = 1e20f;
        uint32_t bs = 0;
        for (uint32_t i = 0; i < 2; i++) {
            float cv = khq_h2f(cents[i * KHQ_D + p * 4 + 3]);
            float dist = fabsf(fmaf(-cv, alpha, v3));
            if (dist < best_s) { best_s = dist; bs = i; }
        }
        d3_code[p] = bs;
        float cvb = khq_h2f(cents[bs * KHQ_D + p * 4 + 3]);
        float resid = fmaf(-cvb, alpha, v3);
        pres[p] = resid;
        if (fabsf(resid) > max_res) max_res = fabsf(resid);
    }
    wr_f32(smeta, max_res);
    float res_scale = fmaxf(max_res, 1e-4f);
    for (int p = 0; p < KHQ_NP; p++) {
        float scaled = fmaf(pres[p] / res_scale, 7.0f, 8.0f);
        d3_dump[p] = (uint32_t)fmaxf(0.0f, fminf(15.0f, roundf(scaled)));
    }
    for (int g = 0; g < 8; g++) {
        uint32_t pv[8];
        for (int i = 0; i < 8; i++) {
            int pid = g * 8 + i;
            pv[i] = (vq_code[pid] & 0x7F) | ((d3_code[pid] & 1) << 7) |
                    ((d3_dump[pid] & 0xF) << 8);
        }
        wr_u32(pay + (g * 3 + 0) * 4, pv[0] | (pv[1] << 12) | ((pv[2] & 0xFF) << 24));
        wr_u32(pay + (g * 3 + 1) * 4,
               (pv[2] >> 8) | (pv[3] << 4) | (pv[4] << 16) | ((pv[5] & 0xF) << 28));
        wr_u32(pay + (g * 3 + 2) * 4, (pv[5] >> 4) | (pv[6] << 8) | (pv[7] << 20));
    }
    uint32_t hl = 0, hh = 0;
    for (int i = 0; i < 32; i++) hl |= ((vq_code[i] >> 7) & 1u) << i;
    for (int i = 0; i < 32; i++) hh |= ((vq_code[32 + i] >> 7) & 1u) << i;
    wr_u32(pay + 24 * 4, hl);
    wr_u32(pay + 25 * 4, hh);
    float st = 0.0f, sv = 0.0f;
    for (int p = 0; p < KHQ_NP; p++) { st += te[p]; sv += ve[p]; }
    *out_rn = khq_f2h(sqrtf(st / (sv + 1e-8f)));
    (void)out_mask_row;
}

/* launch_khq_compress_fp16 semantics (.cu:4279-4310): returns -100 on bad
 * shape.  K rows write mask/norm/rn/payload(40)/smeta=0; V rows write
 * norm/rn/payload(104)/smeta=max_res and leave the mask untouched. */
int khq_ref_compress(const uint16_t* x, const uint16_t* d_vec,
                     const uint16_t* rotor, const uint16_t* cents,
                     const uint16_t* vq, uint32_t* out_mask,
                     uint16_t* out_norms, uint16_t* out_r_norms,
                     uint8_t* out_payload, uint8_t* out_smeta, int n, int d,
                     float ts, float alpha, int is_v) {
    if (n <= 0 || d != KHQ_D) return -100;
    const int stride = is_v ? 104 : 40;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < n; row++)
        compress_row(x + (size_t)row * KHQ_D, d_vec, rotor, cents, vq,
                     out_mask ? out_mask + (size_t)row * 16 : NULL,
                     out_norms + row, out_r_norms + row,
                     out_payload + (size_t)row * stride, out_smeta + (size_t)row * 4,
                     ts, alpha, is_v);
    return 0;
}

/* ------------------------------------------------------- compressed attn */
/* Restates khq_attn_kernel, ref:.cu:1471-1831, for one block
 * (query total_id, split split_id).  The 32-lane warp is emulated with
 * per-lane arrays so that the shuffle reduction order is the reference's. */
typedef struct {
    const uint16_t* q;
    const uint8_t* kpay;
    const uint8_t* vpay;
    const uint8_t* vsm;
    const uint32_t* kmask;
    const uint16_t *knorm, *krn, *vnorm, *vrn;
    const uint16_t *cents_k, *cents_v, *vq, *rotor_k, *rotor_v, *dk, *dv;
    int c_len, h_kv, n_rep, num_queries, num_heads, L_q, start_pos, num_splits;
    float sc, a_k, a_v, rope_base;
} attn_args;

static void attn_block(const attn_args* A, int total_id, int split_id,
                       float* out_base) {
    const int W = 32;
    const int head = total_id / A->L_q;
    const int l_idx = total_id % A->L_q;
    const int hkv = head / A->n_rep;
    const uint16_t* qp = A->q + (size_t)head * 2 * KHQ_D;

    float freqs[32][8];
    float qv[32][8], acc[32][8], kf[32][8];
    float cv0[32][2], cv1[32][2];
    float lcb[32][8], ldk[32][8], rm[32][2][16];
    float cur_c[32][8], cur_s[32][8], st_c[32][8], st_s[32][8];
    for (int t = 0; t < W; t++) {
        for (int j = 0; j < 8; j++) {
            freqs[t][j] = 1.0f;
            if (t < 8) {
                int m = (t & 3) * 8 + j;
                freqs[t][j] = powf(A->rope_base, -2.0f * (float)m / 64.0f);
            }
            qv[t][j] = khq_h2f(qp[t * 8 + j]);
            acc[t][j] = 0.0f;
            int bit = t * 8 + j;
            lcb[t][j] = khq_h2f(A->cents_k[2 * 256 + bit]);
            ldk[t][j] = (1.0f / 256.0f) / (khq_h2f(A->dk[bit]) + 1e-8f);
        }
        for (int p = 0; p < 2; p++) {
            int pid = t * 2 + p;
            cv0[t][p] = khq_h2f(A->cents_v[0 * KHQ_D + pid * 4 + 3]) * A->a_v;
            cv1[t][p] = khq_h2f(A->cents_v[1 * KHQ_D + pid * 4 + 3]) * A->a_v;
            for (int i = 0; i < 16; i++) rm[t][p][i] = khq_h2f(A->rotor_k[pid * 16 + i]);
        }
    }
    int s_limit = (A->L_q > 1) ? (A->c_len < l_idx + 1 ? A->c_len : l_idx + 1) : A->c_len;
    int s_lo = 0, s_hi = s_limit;
    if (A->num_splits > 1) {
        int per = (s_limit + A->num_splits - 1) / A->num_splits;
        s_lo = split_id * per;
        if (s_lo > s_limit) s_lo = s_limit;
        s_hi = s_lo + per;
        if (s_hi > s_limit) s_hi = s_limit;
    }
    for (int t = 0; t < W; t++)
        for (int j = 0; j < 8; j++) {
            float th = (float)(A->start_pos + s_lo) * freqs[t][j];
            cur_c[t][j] = cosf(th);
            cur_s[t][j] = sinf(th);
            st_c[t][j] = cosf(freqs[t][j]);
            st_s[t][j] = sinf(freqs[t][j]);
        }
    float sum_exp = 0.0f, max_s = -1e20f;
    for (int s = s_lo; s < s_hi; s++) {
        if ((s - s_lo) > 0 && (s % 256) == 0) {
            for (int t = 0; t < W; t++)
                for (int j = 0; j < 8; j++) {
                    float th = (float)(A->start_pos + s) * freqs[t][j];
                    cur_c[t][j] = cosf(th);
                    cur_s[t][j] = sinf(th);
                }
        }
        size_t g = (size_t)s * A->h_kv + hkv;
        float nk = khq_h2f(A->knorm[g]);
        float rs = khq_h2f(A->krn[g]);
        const uint8_t* kb = A->kpay + g * 40;
        float mult = (float)rd_u32(kb) / 1000.0f;
        if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
        const uint32_t* mw = A->kmask + g * 16;
        /* K decode .cu:1608-1644 */
        for (int t = 0; t < W; t++) {
            uint32_t base = 0;
            for (int w = 0; w < t / 2; w++) {
                uint32_t m = mw[w];
                base += (uint32_t)__builtin_popcount((m & (m >> 1)) & 0x55555555u);
            }
            if (t % 2 == 1) {
                uint32_t m = mw[t / 2];
                base += (uint32_t)__builtin_popcount((m & (m >> 1)) & 0x00005555u);
            }
            uint32_t lo = base;
            for (int j = 0; j < 8; j++) {
                int bit = t * 8 + j;
                uint32_t code = (mw[bit / 16] >> ((bit % 16) * 2)) & 3u;
                float cbase = lcb[t][j] * mult;
                float kv = 0.0f;
                if (code == 3) {
                    uint32_t jo = lo;
                    float sign = (jo < 50 && ((kb[29 + jo / 8] >> (jo % 8)) & 1)) ? 1.0f : -1.0f;
                    float r4 = (jo < 50) ? (float)((kb[4 + jo / 2] >> ((jo % 2) * 4)) & 0xF) : 0.0f;
                    kv = sign * fmaf(r4, rs, cbase);
                    lo++;
                } else if (code == 2) {
                    kv = cbase;
                } else if (code == 1) {
                    kv = -cbase;
                }
                kf[t][j] = kv * A->a_k * nk;
            }
            /* inverse rotor .cu:1646-1655 */
            float nk8[8];
            for (int p = 0; p < 2; p++)
                for (int c = 0; c < 4; c++) {
                    float a = kf[t][p * 4 + 0] * rm[t][p][c * 4 + 0];
                    a = fmaf(kf[t][p * 4 + 1], rm[t][p][c * 4 + 1], a);
                    a = fmaf(kf[t][p * 4 + 2], rm[t][p][c * 4 + 2], a);
                    a = fmaf(kf[t][p * 4 + 3], rm[t][p][c * 4 + 3], a);
                    nk8[p * 4 + c] = a;
                }
            for (int j = 0; j < 8; j++) kf[t][j] = nk8[j];
            /* in-register FWHT stages .cu:1657-1671 */
            for (int j = 0; j < 8; j += 2) {
                float a = kf[t][j], b = kf[t][j + 1];
                kf[t][j] = a + b; kf[t][j + 1] = a - b;
            }
            for (int b4 = 0; b4 < 8; b4 += 4)
                for (int k = 0; k < 2; k++) {
                    float a = kf[t][b4 + k], b = kf[t][b4 + k + 2];
                    kf[t][b4 + k] = a + b; kf[t][b4 + k + 2] = a - b;
                }
            for (int j = 0; j < 4; j++) {
                float a = kf[t][j], b = kf[t][j + 4];
                kf[t][j] = a + b; kf[t][j + 4] = a - b;
            }
        }
        /* cross-lane FWHT stages .cu:1673-1685 */
        for (int m = 1; m < 32; m <<= 1) {
            float tmp[32][8];
            memcpy(tmp, kf, sizeof(tmp));
            for (int t = 0; t < W; t++) {
                int lower = (t & m) == 0;
                for (int j = 0; j < 8; j++) {
                    float pt = tmp[t ^ m][j];
                    kf[t][j] = lower ? (tmp[t][j] + pt) : (pt - tmp[t][j]);
                }
            }
        }
        for (int t = 0; t < W; t++)
            for (int j = 0; j < 8; j++) kf[t][j] = kf[t][j] * ldk[t][j];
        /* partial RoPE on dims 0..63 (lanes 0..7) .cu:1689-1699 */
        {
            float tmp[32][8];
            memcpy(tmp, kf, sizeof(tmp));
            for (int t = 0; t < 8; t++)
                for (int j = 0; j < 8; j++) {
                    float xo = tmp[t ^ 4][j];
                    float c = cur_c[t][j], sn = cur_s[t][j];
                    if (t < 4) kf[t][j] = fmaf(tmp[t][j], c, -(xo * sn));
                    else kf[t][j] = fmaf(xo, sn, tmp[t][j] * c);
                    cur_c[t][j] = fmaf(c, st_c[t][j], -(sn * st_s[t][j]));
                    cur_s[t][j] = fmaf(sn, st_c[t][j], c * st_s[t][j]);
                }
        }
        /* q.k: per-lane sum then shfl_down tree, lane 0 broadcast */
        float red[32];
        for (int t = 0; t < W; t++) {
            float ps = 0.0f;
            for (int j = 0; j < 8; j++) ps = fmaf(qv[t][j], kf[t][j], ps);
            red[t] = ps;
        }
        for (int off = 16; off > 0; off /= 2) {
            float tmp[32];
            memcpy(tmp, red, sizeof(tmp));
            for (int t = 0; t < W; t++) red[t] = tmp[t] + (t + off < W ? tmp[t + off] : tmp[t]);
        }
        float qk = red[0];
        /* online softmax .cu:1727-1737 */
        float s_val = qk * A->sc;
        float score;
        if (s_val > max_s) {
            float fac = expf(max_s - s_val);
            sum_exp = fmaf(sum_exp, fac, 1.0f);
            for (int t = 0; t < W; t++)
                for (int j = 0; j < 8; j++) acc[t][j] *= fac;
            max_s = s_val;
            score = 1.0f;
        } else {
            float e = expf(s_val - max_s);
            sum_exp += e;
            score = e;
        }
        /* V decode + accumulate in the rotated domain .cu:1739-1762 */
        float nv = khq_h2f(A->vnorm[g]);
        float ec = khq_h2f(A->vrn[g]);
        float smv = rd_f32(A->vsm + g * 4);
        const uint8_t* vp = A->vpay + g * 104;
        uint32_t vhl = rd_u32(vp + 24 * 4), vhh = rd_u32(vp + 25 * 4);
        float pre_v = (A->a_v * nv) * ec;
        float pre_r = smv * nv;
        for (int t = 0; t < W; t++) {
            uint32_t grp = (uint32_t)t / 4;
            uint32_t w0 = rd_u32(vp + (grp * 3 + 0) * 4);
            uint32_t w1 = rd_u32(vp + (grp * 3 + 1) * 4);
            uint32_t w2 = rd_u32(vp + (grp * 3 + 2) * 4);
            uint64_t low64 = ((uint64_t)w1 << 32) | w0;
            uint64_t high64 = ((uint64_t)w2 << 32) | w1;
            for (int p = 0; p < 2; p++) {
                uint32_t pid = (uint32_t)(t * 2 + p);
                uint32_t sub = pid % 8;
                uint32_t pvl = (sub < 4) ? (uint32_t)((low64 >> (sub * 12)) & 0xFFF)
                                         : (uint32_t)((high64 >> ((sub - 4) * 12 + 16)) & 0xFFF);
                uint32_t hb = (pid < 32) ? ((vhl >> pid) & 1) : ((vhh >> (pid - 32)) & 1);
                uint32_t code = (pvl & 0x7F) | (hb << 7);
                uint32_t d3c = (pvl >> 7) & 1;
                uint32_t d3d = (pvl >> 8) & 0xF;
                const uint16_t* cb = A->vq + (size_t)pid * 256 * 3;
                float vv[4];
                for (int k = 0; k < 3; k++) vv[k] = khq_h2f(cb[code * 3 + k]) * pre_v;
                float cvv = d3c == 0 ? cv0[t][p] : cv1[t][p];
                vv[3] = fmaf(((float)d3d - 8.0f) / 7.0f, pre_r, cvv * nv);
                for (int k = 0; k < 4; k++) acc[t][p * 4 + k] = fmaf(score, vv[k], acc[t][p * 4 + k]);
            }
        }
    }
    /* epilogue: inverse V rotor + FWHT + (1/16)/d_v .cu:1776-1826 */
    for (int t = 0; t < W; t++) {
        float nx[8];
        for (int p = 0; p < 2; p++) {
            int pid = t * 2 + p;
            const uint16_t* R = A->rotor_v + pid * 16;
            for (int c = 0; c < 4; c++) {
                float a = acc[t][p * 4 + 0] * khq_h2f(R[c * 4 + 0]);
                a = fmaf(acc[t][p * 4 + 1], khq_h2f(R[c * 4 + 1]), a);
                a = fmaf(acc[t][p * 4 + 2], khq_h2f(R[c * 4 + 2]), a);
                a = fmaf(acc[t][p * 4 + 3], khq_h2f(R[c * 4 + 3]), a);
                nx[p * 4 + c] = a;
            }
        }
        for (int j = 0; j < 8; j++) acc[t][j] = nx[j];
        for (int j = 0; j < 8; j += 2) {
            float a = acc[t][j], b = acc[t][j + 1];
            acc[t][j] = a + b; acc[t][j + 1] = a - b;
        }
        for (int b4 = 0; b4 < 8; b4 += 4)
            for (int k = 0; k < 2; k++) {
                float a = acc[t][b4 + k], b = acc[t][b4 + k + 2];
                acc[t][b4 + k] = a + b; acc[t][b4 + k + 2] = a - b;
            }
        for (int j = 0; j < 4; j++) {
            float a = acc[t][j], b = acc[t][j + 4];
            acc[t][j] = a + b; acc[t][j + 4] = a - b;
        }
    }
    for (int m = 1; m < 32; m <<= 1) {
        float tmp[32][8];
        memcpy(tmp, acc, sizeof(tmp));
        for (int t = 0; t < W; t++) {
            int lower = (t & m) == 0;
            for (int j = 0; j < 8; j++) {
                float pt = tmp[t ^ m][j];
                acc[t][j] = lower ? (tmp[t][j] + pt) : (pt - tmp[t][j]);
            }
        }
    }
    for (int t = 0; t < W; t++)
        for (int j = 0; j < 8; j++)
            out_base[t * 8 + j] = (acc[t][j] * (1.0f / 16.0f)) / (khq_h2f(A->dv[t * 8 + j]) + 1e-8f);
    out_base[KHQ_D] = max_s;
    out_base[KHQ_D + 1] = sum_exp;
}

/* Restates khq_attn_reduce_kernel, ref:.cu:1836-1877. */
static void attn_reduce(const float* partial, float* out, int num_queries,
                        int num_splits) {
    const int stride = KHQ_D + 2;
    for (int q = 0; q < num_queries; q++) {
        const float* base = partial + (size_t)q * num_splits * stride;
        float M = -1e20f;
        for (int sp = 0; sp < num_splits; sp++) {
            float m = base[(size_t)sp * stride + KHQ_D];
            if (m > M) M = m;
        }
        float den = 0.0f;
        for (int sp = 0; sp < num_splits; sp++) {
            const float* p = base + (size_t)sp * stride;
            den = fmaf(p[KHQ_D + 1], expf(p[KHQ_D] - M), den);
        }
        float* o = out + (size_t)q * stride;
        for (int d = 0; d < KHQ_D; d++) {
            float num = 0.0f;
            for (int sp = 0; sp < num_splits; sp++) {
                const float* p = base + (size_t)sp * stride;
                num = fmaf(p[d], expf(p[KHQ_D] - M), num);
            }
            o[d] = num;
        }
        o[KHQ_D] = M;
        o[KHQ_D + 1] = den;
    }
}

/* launch_khq_attn_fp16 semantics, ref:.cu:4314-4375 (h_kv derived as
 * num_heads / n_rep, D fixed at 256, reduce run when num_splits > 1). */
int khq_ref_attn(const uint16_t* q, const uint8_t* k_payload,
                 const uint8_t* v_payload, const uint8_t* v_shared_meta,
                 const uint32_t* k_mask, const uint16_t* k_norms,
                 const uint16_t* k_r_norms, const uint16_t* v_norms,
                 const uint16_t* v_r_norms, const uint16_t* centroids_k,
                 const uint16_t* centroids_v, const uint16_t* vq_centroids,
                 const uint16_t* k_rotor, const uint16_t* v_rotor,
                 const uint16_t* d_vec_k, const uint16_t* d_vec_v,
                 float* out_attn, float* out_partial, int num_queries,
                 int num_heads, int L_q, int c_len, int stride_s, int n_rep,
                 float scale, float alpha_k, float alpha_v, float rope_base,
                 int start_pos, int num_splits) {
    (void)stride_s;
    if (num_queries <= 0 || c_len <= 0) return -100;
    if (num_splits < 1) num_splits = 1;
    if (num_splits > 1 && out_partial == NULL) return -101;
    attn_args A;
    A.q = q; A.kpay = k_payload; A.vpay = v_payload; A.vsm = v_shared_meta;
    A.kmask = k_mask; A.knorm = k_norms; A.krn = k_r_norms; A.vnorm = v_norms;
    A.vrn = v_r_norms; A.cents_k = centroids_k; A.cents_v = centroids_v;
    A.vq = vq_centroids; A.rotor_k = k_rotor; A.rotor_v = v_rotor;
    A.dk = d_vec_k; A.dv = d_vec_v; A.c_len = c_len;
    A.h_kv = n_rep > 0 ? num_heads / n_rep : 1;
    A.n_rep = n_rep; A.num_queries = num_queries; A.num_heads = num_heads;
    A.L_q = L_q; A.start_pos = start_pos; A.num_splits = num_splits;
    A.sc = scale; A.a_k = alpha_k; A.a_v = alpha_v; A.rope_base = rope_base;
    const int stride = KHQ_D + 2;
    const int nblk = num_queries * num_splits;
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < nblk; b++) {
        int tid_q = b / num_splits, sid = b % num_splits;
        if ((tid_q / L_q) >= num_heads) continue;
        float* ob = (num_splits > 1)
                        ? out_partial + ((size_t)tid_q * num_splits + sid) * stride
                        : out_attn + (size_t)tid_q * stride;
        attn_block(&A, tid_q, sid, ob);
    }
    if (num_splits > 1) attn_reduce(out_partial, out_attn, num_queries, num_splits);
    return 0;
}

/* ------------------------------------------------------------- window */
/* Restates khq_window_attn_kernel, ref:.cu:1882-1965 (block 256: q.k summed
 * per 32-lane warp with shfl_down, then warps 0..7 summed in order). */
int khq_ref_window_attn(const uint16_t* q, const uint16_t* ring_k,
                        const uint16_t* ring_v, float* out_attn, int win_start,
                        int win_len, int ring_cap, int H_q, int H_kv, int d,
                        float sc) {
    if (H_q <= 0 || win_len <= 0) return -100;
    const int n_rep = H_q / H_kv;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < H_q; h++) {
        const int hkv = h / n_rep;
        float qv[KHQ_D], acc[KHQ_D];
        for (int i = 0; i < d; i++) { qv[i] = khq_h2f(q[(size_t)h * 2 * d + i]); acc[i] = 0.0f; }
        float sum_exp = 0.0f, max_s = -1e20f;
        for (int s = 0; s < win_len; s++) {
            int slot = (win_start + s) % ring_cap;
            const uint16_t* kr = ring_k + ((size_t)slot * H_kv + hkv) * d;
            const uint16_t* vr = ring_v + ((size_t)slot * H_kv + hkv) * d;
            float warp_tot[8];
            for (int w = 0; w < 8; w++) {
                float lane[32];
                for (int l = 0; l < 32; l++) {
                    int idx = w * 32 + l;
                    lane[l] = idx < d ? qv[idx] * khq_h2f(kr[idx]) : 0.0f;
                }
                for (int off = 16; off > 0; off /= 2) {
                    float tmp[32];
                    memcpy(tmp, lane, sizeof(tmp));
                    for (int l = 0; l < 32; l++) lane[l] = tmp[l] + (l + off < 32 ? tmp[l + off] : tmp[l]);
                }
                warp_tot[w] = lane[0];
            }
            float qk = 0.0f;
            for (int w = 0; w < 8; w++) qk += warp_tot[w];
            float s_val = qk * sc;
            float score;
            if (s_val > max_s) {
                float fac = expf(max_s - s_val);
                sum_exp = fmaf(sum_exp, fac, 1.0f);
                for (int i = 0; i < d; i++) acc[i] *= fac;
                max_s = s_val;
                score = 1.0f;
            } else {
                score = expf(s_val - max_s);
                sum_exp += score;
            }
            for (int i = 0; i < d; i++) acc[i] = fmaf(score, khq_h2f(vr[i]), acc[i]);
        }
        float* o = out_attn + (size_t)h * (d + 2);
        for (int i = 0; i < d; i++) o[i] = acc[i];
        o[d] = max_s;
        o[d + 1] = sum_exp;
    }
    return 0;
}

/* Restates khq_merge_gate_kernel, ref:.cu:1983-2010. */
int khq_ref_merge_gate(const float* attn_c, const float* attn_w,
                       const uint16_t* q_gate, uint16_t* out, int H_q, int d,
                       int has_w) {
    if (H_q <= 0 || d <= 0) return -100;
    for (int h = 0; h < H_q; h++)
        for (int i = 0; i < d; i++) {
            const float* cc = attn_c + (size_t)h * (d + 2);
            float num = cc[i], den = cc[d + 1];
            if (has_w) {
                const float* cw = attn_w + (size_t)h * (d + 2);
                float mc = cc[d], mw = cw[d];
                float M = fmaxf(mc, mw);
                float wc = expf(mc - M), ww = expf(mw - M);
                num = fmaf(num, wc, cw[i] * ww);
                den = fmaf(den, wc, cw[d + 1] * ww);
            }
            float val = num / (den + 1e-8f);
            float g = khq_h2f(q_gate[(size_t)h * 2 * d + d + i]);
            val = val * (1.0f / (1.0f + expf(-g)));
            out[(size_t)h * d + i] = khq_f2h(val);
        }
    return 0;
}

/* Restates khq_gather_q_kernel, ref:.cu:1969-1979. */
int khq_ref_gather_q(const uint16_t* q_gate, uint16_t* q_out, int H_q, int d) {
    if (H_q <= 0 || d <= 0) return -100;
    for (int h = 0; h < H_q; h++)
        for (int i = 0; i < d; i++) q_out[(size_t)h * d + i] = q_gate[(size_t)h * 2 * d + i];
    return 0;
}

/* ------------------------------------------------- config-1 fp16 baseline */
/* Restates partial_rope_sm75_gpu, ref:src/kernels/elementwise_sm75.mojo:1023-1061
 * (half-split pairs (i, i+rot/2), freq = exp(log(theta) * -2i/rot)),
 * applied in place to fp16 rows. */
void khq_ref_partial_rope_fp16(uint16_t* vec, int num_heads, int head_dim,
                               int rotary_dim, int pos, float theta, int stride) {
    int half = rotary_dim / 2;
    int es = stride > 0 ? stride : head_dim;
    for (int h = 0; h < num_heads; h++)
        for (int i = 0; i < half; i++) {
            float ex = -(float)(2 * i) / (float)rotary_dim;
            float fr = expf(logf(theta) * ex);
            float mt = (float)pos * fr;
            float c = cosf(mt), s = sinf(mt);
            float x0 = khq_h2f(vec[(size_t)h * es + i]);
            float x1 = khq_h2f(vec[(size_t)h * es + i + half]);
            vec[(size_t)h * es + i] = khq_f2h(fmaf(x0, c, -(x1 * s)));
            vec[(size_t)h * es + i + half] = khq_f2h(fmaf(x0, s, x1 * c));
        }
}

/* Restates the fp32 host attention of ref:src/models/qwen3_5/attention.mojo:175-196
 * (scores, softmax with 1/Z, P.V, sigmoid gate) over fp16 inputs: q_gate
 * [H_q, 2D] (already roped), k/v cache [seq, H_kv, D] (k already roped). */
void khq_ref_gqa_host(const uint16_t* q_gate, const uint16_t* k_cache,
                      const uint16_t* v_cache, float* out, int seq_len, int H_q,
                      int H_kv, int D, float scale) {
    int grp = H_q / H_kv;
#pragma omp parallel for schedule(static)
    for (int hq = 0; hq < H_q; hq++) {
        int hkv = hq / grp;
        float* sc = (float*)malloc(sizeof(float) * (size_t)seq_len);
        float m = -3.0e38f;
        for (int t = 0; t < seq_len; t++) {
            float dot = 0.0f;
            for (int d = 0; d < D; d++)
                dot = fmaf(khq_h2f(q_gate[(size_t)hq * 2 * D + d]),
                           khq_h2f(k_cache[((size_t)t * H_kv + hkv) * D + d]), dot);
            sc[t] = dot * scale;
            if (sc[t] > m) m = sc[t];
        }
        float z = 0.0f;
        for (int t = 0; t < seq_len; t++) { sc[t] = expf(sc[t] - m); z += sc[t]; }
        for (int t = 0; t < seq_len; t++) sc[t] /= z;
        for (int d = 0; d < D; d++) {
            float acc = 0.0f;
            for (int t = 0; t < seq_len; t++)
                acc = fmaf(sc[t], khq_h2f(v_cache[((size_t)t * H_kv + hkv) * D + d]), acc);
            float g = khq_h2f(q_gate[(size_t)hq * 2 * D + D + d]);
            out[(size_t)hq * D + d] = acc * (1.0f / (1.0f + expf(-g)));
        }
        free(sc);
    }
}

int khq_ref_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void khq_ref_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
