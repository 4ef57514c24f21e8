// khq_attn_mfma.hip -- compressed-region KHQ attention on MI355X matrix cores.
//
// Shape: H_kv = 4 KV heads, 6 query heads per KV head, D = 256.  One
// 256-thread block per token chunk; wavefront w serves KV head w, so a block
// consumes whole 880-byte token records (4 rows x 220 B) and its global
// reads are contiguous.  Tokens are processed in tiles of 16.
//
// The decoded key of row s is   k_s = a_k * norm_s * mult_s * M b_s   with
//   b_s[i] = sgn_i * (cb_i + res_i * rs_s / mult_s)      (code value / scale)
//   M      = diag(1/(256 d)) * H_256 * blockdiag(R_p)    (fixed per layer)
// and RoPE touches only dims 0..63.  The score splits into
//   pass part: q[64:] . (M b)[64:] = t . b,  t = R^T H (q[64:] / (256 d)),
//              t computed once per block (query side), contracted with b on
//              MFMA (t split into fp16 hi + lo rows);
//   roped part: (M b)[0:64] = diag(1/(256 d)) H_64 z,  z_m = sum over the four
//              64-blocks of R b (the first 64 rows of H_256 are [H_64]*4);
//              z = W b on MFMA with the exact fp16 rotor entries as W, then
//              H_64 z on MFMA (z split hi + lo), RoPE in registers, and the
//              dot with q on MFMA (rope'd key split hi + lo).
// b is exact in fp16 for codes 0..2 (+-cb); outlier values are fp16-rounded.
// V is accumulated in the rotated domain as in the reference; its 256
// rotated dims are contracted with the softmax weights on MFMA:
//   dims (p, k<3):  codebook value * (p * a_v * norm * energy)
//   dim  (p, 3):    cents[d3] * (p * a_v * norm) + dump * (p * norm * smeta / 7)
//                   - 8 * sum(p * norm * smeta / 7)
// with the weights split hi + lo.  The inverse V rotor + FWHT + 1/(16 d_v)
// run once per chunk.  Softmax uses a per-head reference maximum that is only
// raised when a tile exceeds it by more than 8 (weights stay <= e^8).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdlib.h>

#include "khq_internal.h"

namespace khq {
namespace mf {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int TT = 16;           // tokens per tile
constexpr int ROWS = TT * 4;     // payload rows per tile (4 KV heads)
constexpr float RESCALE_GAP = 8.0f;

struct __align__(16) Smem {
    _Float16 cb[64 * 256 * 3];           // V codebook (98304 B)
    uint32_t mask[ROWS * 16];            // staged tile
    uint32_t kpay[ROWS * 10];
    uint32_t vpay[ROWS * 26];
    _Float16 knorm[ROWS], krn[ROWS], vnorm[ROWS], vrn[ROWS];
    float vsm[ROWS];
    uint2 sgn[256];                      // mask byte -> 4 fp16 signs {0,-1,+1,0}
    _Float16 cbk[256];                   // cents_k[2]
    float cbkf[256];
    union W {                            // per wavefront scratch
        _Float16 o[TT * 256];            // outlier values, [token][K position]
        _Float16 vt[320 * TT];           // expanded V tile, [column][token]
        float f[6 * 256];                // query transforms / epilogue
    } w[4];
    float pb[4][3][6][TT];               // softmax weights x 3 scalings
};

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float xsh(float v, int m) { return __shfl_xor(v, m, 64); }

// K position (contraction index of the pass/fold MFMAs) -> natural dim.
// kappa = q*16 + b*4 + k  <->  dim = 64 b + 4 q + k  (patch p = 16 b + q).
__device__ __forceinline__ int kdim(int kappa) {
    return ((kappa >> 2) & 3) * 64 + (kappa >> 4) * 4 + (kappa & 3);
}
__device__ __forceinline__ int kpos(int dim) {
    return (((dim >> 2) & 15) << 4) | ((dim >> 6) << 2) | (dim & 3);
}

__device__ __forceinline__ void split(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// FWHT-256 across a wavefront holding 4 consecutive dims per lane.
__device__ __forceinline__ void fwht256(float (&v)[4], int lane) {
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
        for (int c = 0; c < 4; c++) {
            const float p = __shfl_xor(v[c], m, 64);
            v[c] = lower ? (v[c] + p) : (p - v[c]);
        }
    }
}

__global__ __launch_bounds__(256, 1) void attn_mfma_kernel(AttnArgs a, int tiles_per_chunk) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem& S = *reinterpret_cast<Smem*>(smem_raw);
    const int tid = threadIdx.x;
    const int w = tid >> 6;          // KV head
    const int lane = tid & 63;
    const int li = lane & 15;        // token within tile / MFMA row-col index
    const int lg = lane >> 4;        // lane group
    const int chunk = blockIdx.x;
    const int c_len = a.c_len;
    const int s_lo = min(chunk * tiles_per_chunk * TT, c_len);
    const int s_hi = min(s_lo + tiles_per_chunk * TT, c_len);
    const int n_tiles = (s_hi - s_lo + TT - 1) / TT;

    // ------------------------------------------------ per-block tables
    {
        // 96 KB codebook: 24 uint4 per thread, all loads issued before the stores
        const uint4* src = reinterpret_cast<const uint4*>(a.vq);
        uint4* dst = reinterpret_cast<uint4*>(S.cb);
#pragma unroll
        for (int b = 0; b < 3; b++) {
            uint4 tmp[8];
#pragma unroll
            for (int i = 0; i < 8; i++) tmp[i] = src[tid + 256 * (8 * b + i)];
#pragma unroll
            for (int i = 0; i < 8; i++) dst[tid + 256 * (8 * b + i)] = tmp[i];
        }
        const _Float16 one = (_Float16)1.0f, mone = (_Float16)-1.0f, zero = (_Float16)0.0f;
        {
            const int byte = tid;
            h4 s;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int code = (byte >> (2 * c)) & 3;
                s[c] = code == 2 ? one : (code == 1 ? mone : zero);
            }
            S.sgn[byte] = *reinterpret_cast<uint2*>(&s);
        }
        const _Float16 cbv = reinterpret_cast<const _Float16*>(a.cents_k)[512 + tid];
        S.cbk[tid] = cbv;
        S.cbkf[tid] = (float)cbv;
    }

    // ------------------------------------------------ per-wave query side
    // q_h for the 6 heads of KV head w; t_h = R^T H (q[64:] * dks) (pass part)
    const __half* qbase = a.q + (size_t)(w * 6) * 512;
    float* tq = S.w[w].f;  // [6][256]
    float dks[4];
    float rk[16];
#pragma unroll
    for (int c = 0; c < 4; c++) dks[c] = (1.0f / 256.0f) / (__half2float(a.dk[lane * 4 + c]) + 1e-8f);
#pragma unroll
    for (int t = 0; t < 16; t++) rk[t] = __half2float(a.rotor_k[lane * 16 + t]);
    for (int h = 0; h < 6; h++) {
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int dim = lane * 4 + c;
            v[c] = dim >= 64 ? __half2float(qbase[h * 512 + dim]) * dks[c] : 0.0f;
        }
        fwht256(v, lane);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float t = v[0] * rk[0 * 4 + k];
            t = fmaf(v[1], rk[1 * 4 + k], t);
            t = fmaf(v[2], rk[2 * 4 + k], t);
            t = fmaf(v[3], rk[3 * 4 + k], t);
            tq[h * 256 + lane * 4 + k] = t;
        }
    }
    __syncthreads();

    // A operands (rows: 2h = hi, 2h+1 = lo of head h; rows 12..15 zero)
    const int arow_h = li >> 1;
    const bool arow_lo = (li & 1) != 0;
    const bool arow_ok = li < 12;
    h8 At[8];
#pragma unroll
    for (int st = 0; st < 8; st++) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            _Float16 hi = (_Float16)0.0f, lo = (_Float16)0.0f;
            if (arow_ok) split(tq[arow_h * 256 + kdim(32 * st + 8 * lg + e)], hi, lo);
            At[st][e] = arow_lo ? lo : hi;
        }
    }
    // fold: z_(4q+c') = sum_k R_p[c'][k] b_(4p+k) over p = q, q+16, q+32, q+48
    h8 Aw[4][2];
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int st = 2 * T + s;
            const int q_row = 4 * T + (li >> 2), c_row = li & 3;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int kap = 32 * st + 8 * lg + e;
                const int q_col = kap >> 4, b = (kap >> 2) & 3, k = kap & 3;
                const int p = 16 * b + q_col;
                Aw[T][s][e] = (q_row == q_col)
                                  ? reinterpret_cast<const _Float16*>(a.rotor_k)[p * 16 + c_row * 4 + k]
                                  : (_Float16)0.0f;
            }
        }
    // H_64 with 1/(256 d): row j = 16T' + li, K position (kap, lg, e) ->
    // m = 16 (2 (kap & 1) + e / 4) + 4 lg + (e & 3); kap >= 2 is the lo half.
    h8 Ah[4][2];
#pragma unroll
    for (int Tp = 0; Tp < 4; Tp++) {
        const int j = 16 * Tp + li;
        const float dj = (1.0f / 256.0f) / (__half2float(a.dk[j]) + 1e-8f);
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int m = 16 * (2 * kk + (e >> 2)) + 4 * lg + (e & 3);
                const float sgn = (__popc(j & m) & 1) ? -1.0f : 1.0f;
                Ah[Tp][kk][e] = (_Float16)(sgn * dj);
            }
    }
    // q_rot (roped dims 0..63), K positions matching the rope'd key layout
    h8 Aq[2];
#pragma unroll
    for (int kk = 0; kk < 2; kk++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int dim = 16 * (2 * kk + (e >> 2)) + 4 * lg + (e & 3);
            _Float16 hi = (_Float16)0.0f, lo = (_Float16)0.0f;
            if (arow_ok) split(__half2float(qbase[arow_h * 512 + dim]), hi, lo);
            Aq[kk][e] = arow_lo ? lo : hi;
        }

    // RoPE constants: this lane's key dims are 16T' + 4 lg + c' (T' = 0..3),
    // frequency index m = dim & 31 for T' in {0, 1}.
    float fr[8], dc[8], ds[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int m = 16 * (u >> 2) + 4 * lg + (u & 3);
        fr[u] = powf(a.rope_base, -2.0f * (float)m / 64.0f);
        dc[u] = cosf((float)li * fr[u]);
        ds[u] = sinf((float)li * fr[u]);
    }

    // V side per-lane constants (expansion lane = patch `lane`)
    const float av = a.a_v;
    const _Float16 c3v0 = reinterpret_cast<const _Float16*>(a.cents_v)[lane * 4 + 3];
    const _Float16 c3v1 = reinterpret_cast<const _Float16*>(a.cents_v)[256 + lane * 4 + 3];
    const int vgrp = lane >> 3, vsub = lane & 7;
    const int vbit = 12 * vsub;                 // bit offset of the field in the group
    const int vw0 = vgrp * 3 + (vbit >> 5);     // first word holding the field
    const int vsh = vbit & 31;
    const int vhw = 24 + (lane >> 5), vhb = lane & 31;

    // ------------------------------------------------ accumulators
    f4 pv[20];
#pragma unroll
    for (int n = 0; n < 20; n++) pv[n] = f4{0.f, 0.f, 0.f, 0.f};
    float Mref[2] = {-INFINITY, -INFINITY};
    float lsum[2] = {0.f, 0.f}, s3sum[2] = {0.f, 0.f};

    // ------------------------------------------------ tile staging
    const int row0 = s_lo * 4;
    const int rows_valid_total = c_len * 4;
    uint4 pre[5];
    uint2 pre_n = uint2{0, 0};
#define KHQ_PREFETCH(t) \
    do { \
        const int r0 = row0 + (t) * ROWS; \
        const int nvalid = max(0, min(ROWS, rows_valid_total - r0)); \
        /* mask: 64 rows x 64 B = 256 x uint4 -> one per thread */ \
        { \
            const int r = tid >> 2; \
            pre[0] = r < nvalid ? reinterpret_cast<const uint4*>(a.kmask + (size_t)(r0 + r) * 16)[tid & 3] \
                                : uint4{0, 0, 0, 0}; \
        } \
        /* kpay: 64 x 40 B = 160 uint4 */ \
        if (tid < 160) { \
            const int r = (tid * 16) / 40; \
            pre[1] = r < nvalid ? reinterpret_cast<const uint4*>(a.kpay + (size_t)r0 * 40)[tid] \
                                : uint4{0, 0, 0, 0}; \
        } \
        /* vpay: 64 x 104 B = 416 uint4 */ \
        { \
            int i = tid; \
            int r = (i * 16) / 104; \
            pre[2] = r < nvalid ? reinterpret_cast<const uint4*>(a.vpay + (size_t)r0 * 104)[i] \
                                : uint4{0, 0, 0, 0}; \
            i = tid + 256; \
            r = (i * 16) / 104; \
            if (i < 416) \
                pre[3] = r < nvalid ? reinterpret_cast<const uint4*>(a.vpay + (size_t)r0 * 104)[i] \
                                    : uint4{0, 0, 0, 0}; \
        } \
        /* norms: 4 arrays x 16 tokens x 4 rows (uint2 per token); vsm: 16 x uint4 */ \
        if (tid < 64) { \
            const int arr = tid >> 4, part = tid & 15; \
            const __half* base = arr == 0 ? a.knorm : arr == 1 ? a.krn : arr == 2 ? a.vnorm : a.vrn; \
            pre_n = 4 * part < nvalid ? reinterpret_cast<const uint2*>(base + r0)[part] : uint2{0, 0}; \
        } else if (tid < 80) { \
            const int part = tid - 64; \
            pre[4] = 4 * part < nvalid \
                         ? reinterpret_cast<const uint4*>(a.vsm + (size_t)r0 * 4)[part] \
                         : uint4{0, 0, 0, 0}; \
        } \
 \
    } while (0)
#define KHQ_COMMIT() \
    do { \
        reinterpret_cast<uint4*>(S.mask)[tid] = pre[0]; \
        if (tid < 160) reinterpret_cast<uint4*>(S.kpay)[tid] = pre[1]; \
        reinterpret_cast<uint4*>(S.vpay)[tid] = pre[2]; \
        if (tid + 256 < 416) reinterpret_cast<uint4*>(S.vpay)[tid + 256] = pre[3]; \
        if (tid < 64) { \
            const int arr = tid >> 4, part = tid & 15; \
            _Float16* base = arr == 0 ? S.knorm : arr == 1 ? S.krn : arr == 2 ? S.vnorm : S.vrn; \
            reinterpret_cast<uint2*>(base)[part] = pre_n; \
        } else if (tid < 80) { \
            reinterpret_cast<uint4*>(S.vsm)[tid - 64] = pre[4]; \
        } \
 \
    } while (0)
    if (n_tiles > 0) KHQ_PREFETCH(0);
    __syncthreads();
    if (n_tiles > 0) KHQ_COMMIT();
    __syncthreads();

    // RoPE base angle for the first tile, advanced by 16 tokens per tile and
    // re-anchored exactly every 16 tiles.
    float bc[8], bs[8], sc16[8], ss16[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        sc16[u] = cosf(16.0f * fr[u]);
        ss16[u] = sinf(16.0f * fr[u]);
        bc[u] = 1.0f;
        bs[u] = 0.0f;
    }

    _Float16* ow = S.w[w].o;
    _Float16* vt = S.w[w].vt;
    float* pbw = &S.pb[w][0][0][0];

    for (int t = 0; t < n_tiles; t++) {
        const int s0 = s_lo + t * TT;
        if (t + 1 < n_tiles) KHQ_PREFETCH(t + 1);
        if ((t & 15) == 0) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float th = (float)(a.start_pos + s0) * fr[u];
                bc[u] = cosf(th);
                bs[u] = sinf(th);
            }
        }

        // ---- (a) zero outlier buffer
        {
            uint4* o4 = reinterpret_cast<uint4*>(ow);
#pragma unroll
            for (int i = 0; i < (TT * 256 * 2) / 16 / 64; i++) o4[lane + 64 * i] = uint4{0, 0, 0, 0};
        }
        wave_sync();

        // ---- per-token scalars of this lane's token (row li*4 + w)
        const int row = li * 4 + w;
        const uint32_t* krow = &S.kpay[row * 10];
        float mult = (float)krow[0] / 1000.0f;
        if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
        const float nk = (float)S.knorm[row];
        const float rs = (float)S.krn[row];
        const float rr = rs / mult;

        // ---- (b) outliers: lane (token li, quarter lg) owns dims 64 lg .. 64 lg + 63
        {
            const uint32_t* mrow = &S.mask[row * 16 + 4 * lg];
            uint32_t c3[4];
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t m = mrow[i];
                c3[i] = (m & (m >> 1)) & 0x55555555u;
                cnt += __popc(c3[i]);
            }
            // exclusive prefix over the quarters of the same token (lanes li + 16 q)
            int incl = cnt;
            int up = __shfl_up(incl, 16, 64);
            if (lg >= 1) incl += up;
            up = __shfl_up(incl, 32, 64);
            if (lg >= 2) incl += up;
            int j = incl - cnt;
            // compress code-3 flags (even bits) to a 64-bit dim mask
            uint64_t msk = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t x = c3[i];
                x = (x | (x >> 1)) & 0x33333333u;
                x = (x | (x >> 2)) & 0x0F0F0F0Fu;
                x = (x | (x >> 4)) & 0x00FF00FFu;
                x = (x | (x >> 8)) & 0x0000FFFFu;
                msk |= (uint64_t)x << (16 * i);
            }
            const uint64_t signs = ((uint64_t)krow[7] | ((uint64_t)krow[8] << 32)) >> 8;
            const unsigned char* kb = reinterpret_cast<const unsigned char*>(krow);
            _Float16* orow = ow + li * 256;
            while (msk) {
                const int bpos = __builtin_ctzll(msk);
                msk &= msk - 1;
                const int dim = 64 * lg + bpos;
                float sgn = -1.0f, nib = 0.0f;
                if (j < 50) {
                    sgn = ((signs >> j) & 1ull) ? 1.0f : -1.0f;
                    nib = (float)((kb[4 + (j >> 1)] >> ((j & 1) * 4)) & 0xF);
                }
                orow[kpos(dim)] = (_Float16)(sgn * fmaf(nib, rr, S.cbkf[dim]));
                j++;
            }
        }
        wave_sync();

        // ---- (c) b operand + pass / fold MFMAs
        f4 cs = f4{0.f, 0.f, 0.f, 0.f};
        f4 zt[4];
#pragma unroll
        for (int T = 0; T < 4; T++) zt[T] = f4{0.f, 0.f, 0.f, 0.f};
        {
            const unsigned char* mb = reinterpret_cast<const unsigned char*>(&S.mask[row * 16]);
            const _Float16* orow = ow + li * 256;
#pragma unroll
            for (int st = 0; st < 8; st++) {
                const int q = 2 * st + (lg >> 1);
                const int p0 = 32 * (lg & 1) + q, p1 = p0 + 16;
                const uint2 sg0 = S.sgn[mb[p0]];
                const uint2 sg1 = S.sgn[mb[p1]];
                const uint2 cb0 = *reinterpret_cast<const uint2*>(&S.cbk[p0 * 4]);
                const uint2 cb1 = *reinterpret_cast<const uint2*>(&S.cbk[p1 * 4]);
                const h8 ov = *reinterpret_cast<const h8*>(&orow[32 * st + 8 * lg]);
                h4 s0v = *reinterpret_cast<const h4*>(&sg0), s1v = *reinterpret_cast<const h4*>(&sg1);
                h4 c0v = *reinterpret_cast<const h4*>(&cb0), c1v = *reinterpret_cast<const h4*>(&cb1);
                h4 b0 = s0v * c0v, b1 = s1v * c1v;
                h8 bv;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    bv[e] = b0[e] + ov[e];
                    bv[4 + e] = b1[e] + ov[4 + e];
                }
                cs = mfma32(At[st], bv, cs);
                zt[st >> 1] = mfma32(Aw[st >> 1][st & 1], bv, zt[st >> 1]);
            }
        }

        // ---- (d) H_64 (1/(256 d)) on z, split hi + lo
        f4 kr[4];
        {
            h8 zb[4];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int T0 = e >> 2, c = e & 3;
                _Float16 hi, lo;
                split(zt[T0][c], hi, lo);
                zb[0][e] = hi;
                zb[2][e] = lo;
                split(zt[2 + T0][c], hi, lo);
                zb[1][e] = hi;
                zb[3][e] = lo;
            }
#pragma unroll
            for (int Tp = 0; Tp < 4; Tp++) {
                f4 acc = f4{0.f, 0.f, 0.f, 0.f};
                acc = mfma32(Ah[Tp][0], zb[0], acc);
                acc = mfma32(Ah[Tp][1], zb[1], acc);
                acc = mfma32(Ah[Tp][0], zb[2], acc);
                acc = mfma32(Ah[Tp][1], zb[3], acc);
                kr[Tp] = acc;
            }
        }

        // ---- (e) RoPE at absolute position start_pos + s0 + li
        {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float c = fmaf(bc[u], dc[u], -(bs[u] * ds[u]));
                const float s = fmaf(bs[u], dc[u], bc[u] * ds[u]);
                const int T0 = u >> 2, cc = u & 3;
                const float x0 = kr[T0][cc], x1 = kr[T0 + 2][cc];
                kr[T0][cc] = fmaf(x0, c, -(x1 * s));
                kr[T0 + 2][cc] = fmaf(x0, s, x1 * c);
            }
        }

        // ---- (f) roped part of the score on MFMA (key split hi + lo)
        {
            h8 kb[4];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int T0 = e >> 2, c = e & 3;
                _Float16 hi, lo;
                split(kr[T0][c], hi, lo);
                kb[0][e] = hi;
                kb[2][e] = lo;
                split(kr[2 + T0][c], hi, lo);
                kb[1][e] = hi;
                kb[3][e] = lo;
            }
            cs = mfma32(Aq[0], kb[0], cs);
            cs = mfma32(Aq[1], kb[1], cs);
            cs = mfma32(Aq[0], kb[2], cs);
            cs = mfma32(Aq[1], kb[3], cs);
        }

        // ---- (g) scores of heads 2 lg, 2 lg + 1 for token li
        const bool tok_ok = (s0 + li) < s_hi;
        const float fsc = a.a_k * nk * mult * a.sc;
        float sc2[2];
        sc2[0] = tok_ok ? (cs[0] + cs[1]) * fsc : -INFINITY;
        sc2[1] = tok_ok ? (cs[2] + cs[3]) * fsc : -INFINITY;
        if (lg == 3) { sc2[0] = -INFINITY; sc2[1] = -INFINITY; }

        // ---- (h) softmax with a lazily raised reference maximum
        float mx[2];
#pragma unroll
        for (int x = 0; x < 2; x++) {
            float m = sc2[x];
            m = fmaxf(m, xsh(m, 1));
            m = fmaxf(m, xsh(m, 2));
            m = fmaxf(m, xsh(m, 4));
            m = fmaxf(m, xsh(m, 8));
            mx[x] = m;
        }
        const bool need = (mx[0] > Mref[0] + RESCALE_GAP) || (mx[1] > Mref[1] + RESCALE_GAP);
        if (__ballot(need) != 0ull) {
            float fac[2];
#pragma unroll
            for (int x = 0; x < 2; x++) {
                const bool up = mx[x] > Mref[x] + RESCALE_GAP;
                const float nm = up ? mx[x] : Mref[x];
                fac[x] = (nm == -INFINITY) ? 1.0f : expf(Mref[x] - nm);
                Mref[x] = nm;
                lsum[x] *= fac[x];
                s3sum[x] *= fac[x];
            }
#pragma unroll
            for (int n = 0; n < 20; n++) {
                pv[n][0] *= fac[0];
                pv[n][1] *= fac[0];
                pv[n][2] *= fac[1];
                pv[n][3] *= fac[1];
            }
        }
        float pr[2];
#pragma unroll
        for (int x = 0; x < 2; x++) {
            pr[x] = (sc2[x] == -INFINITY) ? 0.0f : expf(sc2[x] - Mref[x]);
            lsum[x] += pr[x];
        }

        // ---- (i) weights x V scalings -> A operands (rows = head hi/lo, K = tokens)
        {
            const float nv = (float)S.vnorm[row];
            const float en = (float)S.vrn[row];
            const float smv = S.vsm[row];
            const float sv0 = (av * nv) * en;
            const float sv1 = av * nv;
            const float sv2 = nv * smv / 7.0f;
            if (lg < 3) {
#pragma unroll
                for (int x = 0; x < 2; x++) {
                    const int h = 2 * lg + x;
                    pbw[(0 * 6 + h) * TT + li] = pr[x] * sv0;
                    pbw[(1 * 6 + h) * TT + li] = pr[x] * sv1;
                    const float p2 = pr[x] * sv2;
                    pbw[(2 * 6 + h) * TT + li] = p2;
                    s3sum[x] += p2;
                }
            }
        }
        wave_sync();
        h4 Ap[3];
#pragma unroll
        for (int v = 0; v < 3; v++) {
            const f4 pw = arow_ok ? *reinterpret_cast<const f4*>(&pbw[(v * 6 + arow_h) * TT + 4 * lg])
                                  : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 hi, lo;
                split(pw[e], hi, lo);
                Ap[v][e] = arow_lo ? lo : hi;
            }
        }

        // ---- (j) expand the V tile: lane = patch, columns 3p+k, 192+p, 256+p
        {
#pragma unroll
            for (int quad = 0; quad < 4; quad++) {
                h4 col[5];
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int tok = quad * 4 + tt;
                    const uint32_t* vr = &S.vpay[(tok * 4 + w) * 26];
                    const uint64_t pair = (uint64_t)vr[vw0] | ((uint64_t)vr[vw0 + 1 < 26 ? vw0 + 1 : vw0] << 32);
                    const uint32_t fld = (uint32_t)(pair >> vsh) & 0xFFFu;
                    const uint32_t code = (fld & 0x7Fu) | (((vr[vhw] >> vhb) & 1u) << 7);
                    const _Float16* ce = &S.cb[(lane * 256 + code) * 3];
                    col[0][tt] = ce[0];
                    col[1][tt] = ce[1];
                    col[2][tt] = ce[2];
                    col[3][tt] = ((fld >> 7) & 1u) ? c3v1 : c3v0;
                    col[4][tt] = (_Float16)(float)((fld >> 8) & 0xFu);
                }
                *reinterpret_cast<h4*>(&vt[(3 * lane + 0) * TT + 4 * quad]) = col[0];
                *reinterpret_cast<h4*>(&vt[(3 * lane + 1) * TT + 4 * quad]) = col[1];
                *reinterpret_cast<h4*>(&vt[(3 * lane + 2) * TT + 4 * quad]) = col[2];
                *reinterpret_cast<h4*>(&vt[(192 + lane) * TT + 4 * quad]) = col[3];
                *reinterpret_cast<h4*>(&vt[(256 + lane) * TT + 4 * quad]) = col[4];
            }
        }
        wave_sync();

        // ---- (k) P x V on MFMA (16x16x16, K = the 16 tokens)
#pragma unroll
        for (int n = 0; n < 20; n++) {
            const h4 bv = *reinterpret_cast<const h4*>(&vt[(16 * n + li) * TT + 4 * lg]);
            pv[n] = mfma16(Ap[n < 12 ? 0 : (n < 16 ? 1 : 2)], bv, pv[n]);
        }

        // ---- (l) advance RoPE base by 16 tokens, stage the next tile
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float nc = fmaf(bc[u], sc16[u], -(bs[u] * ss16[u]));
            const float ns = fmaf(bs[u], sc16[u], bc[u] * ss16[u]);
            bc[u] = nc;
            bs[u] = ns;
        }
        __syncthreads();
        if (t + 1 < n_tiles) KHQ_COMMIT();
        __syncthreads();
    }

    // ------------------------------------------------ epilogue
    // sums over the 16 tokens (lanes) of each head group
#pragma unroll
    for (int x = 0; x < 2; x++) {
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) {
            lsum[x] += xsh(lsum[x], m);
            s3sum[x] += xsh(s3sum[x], m);
        }
    }
    float* ep = S.w[w].f;  // [6][256] rotated-domain accumulators
    if (lg < 3) {
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const int h = 2 * lg + x;
#pragma unroll
            for (int n = 0; n < 12; n++) {
                const int col = 16 * n + li;
                ep[h * 256 + 4 * (col / 3) + col % 3] = pv[n][2 * x] + pv[n][2 * x + 1];
            }
#pragma unroll
            for (int n = 12; n < 16; n++) {
                const int p = 16 * (n - 12) + li;
                const float d3 = pv[n][2 * x] + pv[n][2 * x + 1];
                const float du = pv[n + 4][2 * x] + pv[n + 4][2 * x + 1];
                ep[h * 256 + 4 * p + 3] = d3 + du - 8.0f * s3sum[x];
            }
        }
    }
    // head group lg holds Mref / lsum of heads 2 lg, 2 lg + 1: publish via LDS
    __shared__ float s_ml[4][6][2];
    if (li == 0 && lg < 3) {
#pragma unroll
        for (int x = 0; x < 2; x++) {
            s_ml[w][2 * lg + x][0] = Mref[x];
            s_ml[w][2 * lg + x][1] = lsum[x];
        }
    }
    __syncthreads();
    float rv[16];
#pragma unroll
    for (int t = 0; t < 16; t++) rv[t] = __half2float(a.rotor_v[lane * 16 + t]);
    for (int h = 0; h < 6; h++) {
        float o[4], u[4];
#pragma unroll
        for (int c = 0; c < 4; c++) o[c] = ep[h * 256 + lane * 4 + c];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float t = o[0] * rv[c * 4 + 0];
            t = fmaf(o[1], rv[c * 4 + 1], t);
            t = fmaf(o[2], rv[c * 4 + 2], t);
            t = fmaf(o[3], rv[c * 4 + 3], t);
            u[c] = t;
        }
        fwht256(u, lane);
        const int hq = w * 6 + h;
        float* out = a.part + ((size_t)hq * a.part_stride + a.part_offset + chunk) * 258;
        const float M = s_ml[w][h][0];
        const float L = s_ml[w][h][1];
        const bool empty = (M == -INFINITY);
#pragma unroll
        for (int c = 0; c < 4; c++)
            out[lane * 4 + c] =
                empty ? 0.0f : (u[c] * (1.0f / 16.0f)) / (__half2float(a.dv[lane * 4 + c]) + 1e-8f);
        if (lane == 0) {
            out[256] = empty ? -1e20f : M;
            out[257] = empty ? 0.0f : L;
        }
    }
}

}  // namespace mf

size_t attn_mfma_smem_bytes() { return sizeof(mf::Smem); }

int attn_mfma_tiles_per_chunk(int c_len, int* n_chunks) {
    static const int max_chunks = [] {
        const char* e = getenv("KHQ_MFMA_MAX_CHUNKS");
        const int v = e ? atoi(e) : 0;
        return v > 0 ? v : 256;
    }();
    const int tiles = (c_len + mf::TT - 1) / mf::TT;
    int chunks = tiles < max_chunks ? tiles : max_chunks;
    if (chunks < 1) chunks = 1;
    const int per = (tiles + chunks - 1) / chunks;
    *n_chunks = (tiles + per - 1) / per;
    return per;
}

hipError_t launch_attn_mfma(const AttnArgs& a, int tiles_per_chunk, int n_chunks,
                            hipStream_t st) {
    static bool configured = false;
    const size_t smem = sizeof(mf::Smem);
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&mf::attn_mfma_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(mf::attn_mfma_kernel, dim3(n_chunks), dim3(256), smem, st, a,
                       tiles_per_chunk);
    return hipGetLastError();
}

}  // namespace khq
