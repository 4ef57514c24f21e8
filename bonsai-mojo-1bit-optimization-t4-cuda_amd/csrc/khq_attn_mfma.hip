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

#ifdef KHQ_PHASE_TIMING
__device__ unsigned long long phase_cycles[16];
#define PHASE(k)                                                              \
    do {                                                                      \
        const unsigned long long now_ = __builtin_amdgcn_s_memtime();         \
        if (blockIdx.x == 0 && threadIdx.x == 0) phase_cycles[k] += now_ - ph_t; \
        ph_t = now_;                                                          \
    } while (0)
#else
#define PHASE(k) do { } while (0)
#endif

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int TT = 16;           // tokens per tile
constexpr int ROWS = TT * 4;     // payload rows per tile (4 KV heads)
constexpr float RESCALE_GAP = 8.0f;

// Padded strides (in 32-bit words) keep the 16 tokens of a tile, and the 64
// codebook patches, in different LDS banks.
constexpr int MASK_TS = 68;    // 4 rows x 16 words + 4
constexpr int KPAY_TS = 44;    // 4 rows x 10 words + 4
constexpr int VPAY_TS = 108;   // 4 rows x 26 words + 4
constexpr int CB_PS = 770;     // halves per codebook patch (768 + 2)
constexpr int O_TS = 264;      // halves per token of the outlier buffer
constexpr int VT_CS = 20;      // halves per V-tile column (16 tokens + 4)
constexpr int VT_COLS = 160;   // V-tile columns per half (32 patches x 5)

struct __align__(16) Smem {
    _Float16 cb[64 * CB_PS];             // V codebook (98560 B)
    uint32_t mask[TT * MASK_TS];         // staged tile
    uint32_t kpay[TT * KPAY_TS];
    uint32_t vpay[TT * VPAY_TS];
    _Float16 knorm[ROWS], krn[ROWS], vnorm[ROWS], vrn[ROWS];
    float vsm[ROWS];
    uint2 sgn[256];                      // mask byte -> 4 fp16 signs {0,-1,+1,0}
    _Float16 cbk[256];                   // cents_k[2]
    union W {                            // per wavefront scratch
        _Float16 o[TT * O_TS];           // outlier values, [token][dim]
        _Float16 vt[VT_COLS * VT_CS];    // expanded V tile, [column][token]
        float f[6 * 256];                // query transforms / epilogue
    } w[4];
    float pb[4][3][6][TT];               // softmax weights x 3 scalings
    float rope[4][3][8];                 // per lane group: freq, cos(16 f), sin(16 f)
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

// Cross-lane moves inside a 16-lane row (DPP, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// max / sum over the 16 lanes of a row: xor 1, xor 2 (quad_perm), then
// row_half_mirror and row_mirror fold the quads and the half rows.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}

// K position (contraction index of the pass/fold MFMAs) -> natural dim.
// kappa = q*16 + b*4 + k  <->  dim = 64 b + 4 q + k  (patch p = 16 b + q).
__device__ __forceinline__ int kdim(int kappa) {
    return ((kappa >> 2) & 3) * 64 + (kappa >> 4) * 4 + (kappa & 3);
}
__device__ __forceinline__ int kpos(int dim) {
    return (((dim >> 2) & 15) << 4) | ((dim >> 6) << 2) | (dim & 3);
}

// cos / sin of an fp32 angle (radians): exact reduction to [-1/2, 1/2]
// revolutions in fp64, then the hardware sine/cosine (revolution input).
__device__ __forceinline__ void sincos_rev(float th, float& c, float& s) {
    double r = (double)th * 0.15915494309189535;  // 1 / (2 pi)
    r -= rint(r);
    const float rf = (float)r;
    c = __builtin_amdgcn_cosf(rf);
    s = __builtin_amdgcn_sinf(rf);
}

__device__ __forceinline__ float fexp(float x) { return __expf(x); }

// hi + lo fp16 split of two floats (hi truncated, lo carries the rest).
__device__ __forceinline__ void split2(float x, float y, _Float16& xh, _Float16& yh,
                                       _Float16& xl, _Float16& yl) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x, y));
    const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x - (float)hi[0], y - (float)hi[1]));
    xh = hi[0];
    yh = hi[1];
    xl = lo[0];
    yl = lo[1];
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
#ifdef KHQ_PHASE_TIMING
    unsigned long long ph_t = __builtin_amdgcn_s_memtime();
#endif
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
        // 96 KB codebook: 24 uint4 per thread, all loads issued before the stores;
        // patch p lands at word p * CB_PS / 2 (96 uint4 per patch)
        const uint4* src = reinterpret_cast<const uint4*>(a.vq);
        uint32_t* dst = reinterpret_cast<uint32_t*>(S.cb);
#pragma unroll
        for (int b = 0; b < 3; b++) {
            uint4 tmp[8];
#pragma unroll
            for (int i = 0; i < 8; i++) tmp[i] = src[tid + 256 * (8 * b + i)];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = tid + 256 * (8 * b + i);
                uint32_t* d = dst + (c / 96) * (CB_PS / 2) + (c % 96) * 4;
                d[0] = tmp[i].x;
                d[1] = tmp[i].y;
                d[2] = tmp[i].z;
                d[3] = tmp[i].w;
            }
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
    }

    // ------------------------------------------------ per-wave query side
    // q_h for the 6 heads of KV head w; t_h = R^T H (q[64:] * dks) (pass part).
    // H_256 = H_16 (x) H_16 (dim = 16 hi + lo): rows then columns in LDS.
    const __half* qbase = a.q + (size_t)(w * 6) * 512;
    float* tq = S.w[w].f;  // [6][256]
    {
        float dks[4];
#pragma unroll
        for (int c = 0; c < 4; c++)
            dks[c] = (1.0f / 256.0f) / (__half2float(a.dk[lane * 4 + c]) + 1e-8f);
#pragma unroll
        for (int h = 0; h < 6; h++) {
            const uint2 qr = *reinterpret_cast<const uint2*>(qbase + h * 512 + lane * 4);
            const __half* qh = reinterpret_cast<const __half*>(&qr);
            f4 v;
#pragma unroll
            for (int c = 0; c < 4; c++) v[c] = lane >= 16 ? __half2float(qh[c]) * dks[c] : 0.0f;
            *reinterpret_cast<f4*>(&tq[h * 256 + lane * 4]) = v;
        }
        wave_sync();
        // 96 transforms of 16 points (6 heads x 16), first along lo then along hi
#pragma unroll
        for (int pass = 0; pass < 2; pass++) {
            for (int item = lane; item < 96; item += 64) {
                const int h = item >> 4, r = item & 15;
                const int base = h * 256 + (pass == 0 ? r * 16 : r);
                const int step = pass == 0 ? 1 : 16;
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = tq[base + i * step];
#pragma unroll
                for (int m = 1; m < 16; m <<= 1)
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        if ((i & m) == 0) {
                            const float x = v[i], y = v[i + m];
                            v[i] = x + y;
                            v[i + m] = x - y;
                        }
#pragma unroll
                for (int i = 0; i < 16; i++) tq[base + i * step] = v[i];
            }
            wave_sync();
        }
        // per patch: t[4p + k] = sum_c u[4p + c] R_p[c][k]
        float rk[16];
        {
            const uint4* rp = reinterpret_cast<const uint4*>(a.rotor_k + lane * 16);
            const uint4 r0 = rp[0], r1 = rp[1];
            const __half* rh0 = reinterpret_cast<const __half*>(&r0);
            const __half* rh1 = reinterpret_cast<const __half*>(&r1);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                rk[t] = __half2float(rh0[t]);
                rk[8 + t] = __half2float(rh1[t]);
            }
        }
#pragma unroll
        for (int h = 0; h < 6; h++) {
            const f4 u = *reinterpret_cast<const f4*>(&tq[h * 256 + lane * 4]);
            f4 t;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float x = u[0] * rk[0 * 4 + k];
                x = fmaf(u[1], rk[1 * 4 + k], x);
                x = fmaf(u[2], rk[2 * 4 + k], x);
                x = fmaf(u[3], rk[3 * 4 + k], x);
                t[k] = x;
            }
            *reinterpret_cast<f4*>(&tq[h * 256 + lane * 4]) = t;
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
    // fold: z_(4q+c') = sum_k R_p[c'][k] b_(4p+k) over p = q, q+16, q+32, q+48.
    // In M-tile T only K-step 2T + s_fold carries this lane's row (q_row = q_col
    // needs li/4 = 2 s + lg/2); Aw[T] holds those 8 rotor entries.
    {   // stage rotor_k (2 KB) in the V staging area, free until the first commit
        const uint4* src = reinterpret_cast<const uint4*>(a.rotor_k);
        if (tid < 128) reinterpret_cast<uint4*>(S.vpay)[tid] = src[tid];
        __syncthreads();
    }
    const _Float16* rk_lds = reinterpret_cast<const _Float16*>(S.vpay);
    const int s_fold = ((li >> 2) - (lg >> 1)) >> 1;
    const bool fold_ok = (((li >> 2) - (lg >> 1)) & 1) == 0 && s_fold >= 0 && s_fold < 2;
    h8 Aw[4];
#pragma unroll
    for (int T = 0; T < 4; T++) {
        const int c_row = li & 3;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int b = 2 * (lg & 1) + (e >> 2), k = e & 3;
            const int p = 16 * b + 4 * T + (li >> 2);
            Aw[T][e] = fold_ok ? rk_lds[p * 16 + c_row * 4 + k] : (_Float16)0.0f;
        }
    }
    const h8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
    // H_64 = H_4 (x) H_16 (j = 16 T' + li, m = 16 T + 4 lg + c'):
    // A[T'][kk] = H_4[T'][2 kk + e/4] * H_16[li][4 lg + (e & 3)] / 256; the
    // sign of 1/d_j is applied to the output rows instead.  Ag[0] = [g, g],
    // Ag[1] = [g, -g], with -Ag for the negated patterns.
    h8 Ag[2];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float g = ((__popc(li & (4 * lg + (e & 3))) & 1) ? -1.0f : 1.0f) / 256.0f;
        Ag[0][e] = (_Float16)g;
        Ag[1][e] = (_Float16)((e >> 2) ? -g : g);
    }
    // output-row signs of 1/d for this lane's rows j = 16 T' + 4 lg + c'
    float dsg[4][4];
#pragma unroll
    for (int Tp = 0; Tp < 4; Tp++)
#pragma unroll
        for (int c = 0; c < 4; c++)
            dsg[Tp][c] = (__half2float(a.dk[16 * Tp + 4 * lg + c]) < 0.0f) ? -1.0f : 1.0f;
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
    float dc[8], ds[8];
    if (w == 0 && li < 8) {  // lanes (u = li, lg) of wave 0 fill the group table
        const int u = li;
        const int m = 16 * (u >> 2) + 4 * lg + (u & 3);
        const float f = powf(a.rope_base, -2.0f * (float)m / 64.0f);
        S.rope[lg][0][u] = f;
        S.rope[lg][1][u] = cosf(16.0f * f);
        S.rope[lg][2][u] = sinf(16.0f * f);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; u++) sincos_rev((float)li * S.rope[lg][0][u], dc[u], ds[u]);

    // V side per-lane constants (expansion lane = patch `lane`)
    const float av = a.a_v;
    const _Float16* cvh = reinterpret_cast<const _Float16*>(a.cents_v);
    const _Float16 c3v0a = cvh[(lane & 31) * 4 + 3], c3v1a = cvh[256 + (lane & 31) * 4 + 3];
    const _Float16 c3v0b = cvh[(32 + (lane & 31)) * 4 + 3], c3v1b = cvh[256 + (32 + (lane & 31)) * 4 + 3];

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
        *reinterpret_cast<uint4*>(&S.mask[(tid >> 4) * MASK_TS + (tid & 15) * 4]) = pre[0]; \
        if (tid < 160) \
            *reinterpret_cast<uint4*>(&S.kpay[(tid / 10) * KPAY_TS + (tid % 10) * 4]) = pre[1]; \
        *reinterpret_cast<uint4*>(&S.vpay[(tid / 26) * VPAY_TS + (tid % 26) * 4]) = pre[2]; \
        if (tid + 256 < 416) \
            *reinterpret_cast<uint4*>(&S.vpay[((tid + 256) / 26) * VPAY_TS + ((tid + 256) % 26) * 4]) = \
                pre[3]; \
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

    // RoPE base angle of the tile, advanced by 16 tokens per tile and
    // re-anchored exactly every 16 tiles.
    float bc[8], bs[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        bc[u] = 1.0f;
        bs[u] = 0.0f;
    }

    PHASE(0);
    _Float16* ow = S.w[w].o;
    _Float16* vt = S.w[w].vt;
    float* pbw = &S.pb[w][0][0][0];

    for (int t = 0; t < n_tiles; t++) {
        const int s0 = s_lo + t * TT;
        if (t + 1 < n_tiles) KHQ_PREFETCH(t + 1);
        if ((t & 15) == 0) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float th = (float)(a.start_pos + s0) * S.rope[lg][0][u];
                sincos_rev(th, bc[u], bs[u]);
            }
        }

        // ---- (a) zero outlier buffer
        {
            uint4* o4 = reinterpret_cast<uint4*>(ow);
            for (int i = lane; i < (TT * O_TS * 2) / 16; i += 64) o4[i] = uint4{0, 0, 0, 0};
        }
        wave_sync();

        PHASE(1);
        // ---- per-token scalars of this lane's token (row li*4 + w)
        const int row = li * 4 + w;
        const uint32_t* krow = &S.kpay[li * KPAY_TS + w * 10];
        float mult = (float)krow[0] / 1000.0f;
        if (mult < 0.1f || mult > 10.0f || isnan(mult)) mult = 1.0f;
        const float nk = (float)S.knorm[row];
        const float rs = (float)S.krn[row];
        const float rr = rs / mult;

        // ---- (b) outliers: lane (token li, quarter lg) owns dims 64 lg .. 64 lg + 63
        {
            const uint32_t* mrow = &S.mask[li * MASK_TS + w * 16 + 4 * lg];
            uint32_t c3[4], c3w[4];
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t m = mrow[i];
                c3w[i] = m;
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
            // sign bits (bytes 29..35) and nibbles (bytes 4..28), both in outlier order;
            // only ordinals < 50 are stored (others: sign -1, residual 0).  The
            // sign goes back into the staged mask (code 3 -> 2 for +, 1 for -),
            // so the b operand's sign table yields +-cb; O keeps the signed
            // residual nib * rs / mult.
            const uint64_t signs = ((uint64_t)krow[7] | ((uint64_t)krow[8] << 32)) >> 8;
            const int nv0 = max(0, min(64, 50 - j));
            uint64_t sw = (j < 64 ? (signs >> j) : 0ull) & (nv0 >= 64 ? ~0ull : ((1ull << nv0) - 1ull));
            uint64_t nw = 0, neg = 0;
            int left = 0;  // nibbles remaining in nw
            const uint64_t all3 = msk;
            _Float16* orow = ow + li * O_TS + 64 * lg;
            while (msk) {
                if (left == 0) {
                    // 16 nibbles from ordinal j: bit 32 + 4 j of the row (dword 1 + j / 8)
                    const int dwi = 1 + (j >> 3), sh = 4 * (j & 7);
                    const uint64_t lo64 = (uint64_t)krow[min(dwi, 9)] | ((uint64_t)krow[min(dwi + 1, 9)] << 32);
                    const uint32_t d2 = krow[min(dwi + 2, 9)];
                    nw = (lo64 >> sh) | (sh ? ((uint64_t)d2 << (64 - sh)) : 0ull);
                    const int nvn = max(0, min(16, 50 - j));
                    nw &= (nvn >= 16) ? ~0ull : ((1ull << (4 * nvn)) - 1ull);
                    left = 16;
                }
                const int bpos = __builtin_ctzll(msk);
                msk &= msk - 1;
                const float r = (float)(uint32_t)(nw & 15ull) * rr;
                const bool pos = (sw & 1ull) != 0ull;
                orow[bpos] = (_Float16)(pos ? r : -r);
                neg |= (uint64_t)(!pos) << bpos;
                nw >>= 4;
                sw >>= 1;
                left--;
                j++;
            }
            // spread the 16-bit halves back to the 2-bit code positions
            uint32_t* mw = &S.mask[li * MASK_TS + w * 16 + 4 * lg];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t ng = (uint32_t)(neg >> (16 * i)) & 0xFFFFu;
                uint32_t a3 = (uint32_t)(all3 >> (16 * i)) & 0xFFFFu;
                ng = (ng | (ng << 8)) & 0x00FF00FFu;
                ng = (ng | (ng << 4)) & 0x0F0F0F0Fu;
                ng = (ng | (ng << 2)) & 0x33333333u;
                ng = (ng | (ng << 1)) & 0x55555555u;
                a3 = (a3 | (a3 << 8)) & 0x00FF00FFu;
                a3 = (a3 | (a3 << 4)) & 0x0F0F0F0Fu;
                a3 = (a3 | (a3 << 2)) & 0x33333333u;
                a3 = (a3 | (a3 << 1)) & 0x55555555u;
                // negative: clear bit 1 (3 -> 1); positive: clear bit 0 (3 -> 2)
                mw[i] = c3w[i] ^ ((ng << 1) | (a3 & ~ng));
            }
        }
        wave_sync();

        PHASE(2);
        // ---- (c) b operand + pass / fold MFMAs
        f4 cs = f4{0.f, 0.f, 0.f, 0.f};
        f4 zt[4];
#pragma unroll
        for (int T = 0; T < 4; T++) zt[T] = f4{0.f, 0.f, 0.f, 0.f};
        {
            const unsigned char* mb = reinterpret_cast<const unsigned char*>(&S.mask[li * MASK_TS + w * 16]);
            const _Float16* orow = ow + li * O_TS;
#pragma unroll
            for (int st = 0; st < 8; st++) {
                const int q = 2 * st + (lg >> 1);
                const int p0 = 32 * (lg & 1) + q, p1 = p0 + 16;
                const uint2 sg0 = S.sgn[mb[p0]];
                const uint2 sg1 = S.sgn[mb[p1]];
                const uint2 cb0 = *reinterpret_cast<const uint2*>(&S.cbk[p0 * 4]);
                const uint2 cb1 = *reinterpret_cast<const uint2*>(&S.cbk[p1 * 4]);
                const h4 ov0 = *reinterpret_cast<const h4*>(&orow[4 * p0]);
                const h4 ov1 = *reinterpret_cast<const h4*>(&orow[4 * p1]);
                h4 s0v = *reinterpret_cast<const h4*>(&sg0), s1v = *reinterpret_cast<const h4*>(&sg1);
                h4 c0v = *reinterpret_cast<const h4*>(&cb0), c1v = *reinterpret_cast<const h4*>(&cb1);
                const h4 b0 = s0v * c0v + ov0, b1 = s1v * c1v + ov1;
                const h8 bv = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
                cs = mfma32(At[st], bv, cs);
                zt[st >> 1] = mfma32((st & 1) == s_fold ? Aw[st >> 1] : hzero, bv, zt[st >> 1]);
            }
        }

        PHASE(3);
        // ---- (d) H_64 (1/(256 d)) on z, split hi + lo
        f4 kr[4];
        {
            h8 zb[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const int T0 = e >> 2, c = e & 3;
                _Float16 a0, a1, a2, a3;
                split2(zt[T0][c], zt[T0][c + 1], a0, a1, a2, a3);
                zb[0][e] = a0; zb[0][e + 1] = a1; zb[2][e] = a2; zb[2][e + 1] = a3;
                split2(zt[2 + T0][c], zt[2 + T0][c + 1], a0, a1, a2, a3);
                zb[1][e] = a0; zb[1][e + 1] = a1; zb[3][e] = a2; zb[3][e + 1] = a3;
            }
            // H_4 rows: T'=0 [+ + + +], 1 [+ - + -], 2 [+ + - -], 3 [+ - - +]
            // over T = 0..3 = (kk, half): Ag[0] = [+,+], Ag[1] = [+,-].
            const h8 A00 = Ag[0], A01 = Ag[1], A10 = -Ag[0], A11 = -Ag[1];
#pragma unroll
            for (int Tp = 0; Tp < 4; Tp++) {
                const h8 k0 = (Tp & 1) ? A01 : A00;               // T = 0, 1
                const h8 k1 = (Tp == 0) ? A00 : (Tp == 1) ? A01 : (Tp == 2) ? A10 : A11;  // T = 2, 3
                f4 acc = f4{0.f, 0.f, 0.f, 0.f};
                acc = mfma32(k0, zb[0], acc);
                acc = mfma32(k1, zb[1], acc);
                acc = mfma32(k0, zb[2], acc);
                acc = mfma32(k1, zb[3], acc);
#pragma unroll
                for (int c = 0; c < 4; c++) acc[c] *= dsg[Tp][c];
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
            for (int e = 0; e < 8; e += 2) {
                const int T0 = e >> 2, c = e & 3;
                _Float16 a0, a1, a2, a3;
                split2(kr[T0][c], kr[T0][c + 1], a0, a1, a2, a3);
                kb[0][e] = a0; kb[0][e + 1] = a1; kb[2][e] = a2; kb[2][e + 1] = a3;
                split2(kr[2 + T0][c], kr[2 + T0][c + 1], a0, a1, a2, a3);
                kb[1][e] = a0; kb[1][e + 1] = a1; kb[3][e] = a2; kb[3][e + 1] = a3;
            }
            cs = mfma32(Aq[0], kb[0], cs);
            cs = mfma32(Aq[1], kb[1], cs);
            cs = mfma32(Aq[0], kb[2], cs);
            cs = mfma32(Aq[1], kb[3], cs);
        }

        PHASE(4);
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
            mx[x] = row16_max(sc2[x]);
        }
        const bool need = (mx[0] > Mref[0] + RESCALE_GAP) || (mx[1] > Mref[1] + RESCALE_GAP);
        if (__ballot(need) != 0ull) {
            float fac[2];
#pragma unroll
            for (int x = 0; x < 2; x++) {
                const bool up = mx[x] > Mref[x] + RESCALE_GAP;
                const float nm = up ? mx[x] : Mref[x];
                fac[x] = (nm == -INFINITY) ? 1.0f : fexp(Mref[x] - nm);
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
            pr[x] = (sc2[x] == -INFINITY) ? 0.0f : fexp(sc2[x] - Mref[x]);
            lsum[x] += pr[x];
        }

        PHASE(5);
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
            for (int e = 0; e < 4; e += 2) {
                _Float16 h0, h1, l0, l1;
                split2(pw[e], pw[e + 1], h0, h1, l0, l1);
                Ap[v][e] = arow_lo ? l0 : h0;
                Ap[v][e + 1] = arow_lo ? l1 : h1;
            }
        }

        PHASE(6);
        // ---- (j, k) V in two halves of 32 patches: expand [160 columns][16 tokens]
        // (column 3p'+k: codebook dim k of patch p'; 96+p': cents[d3]; 128+p': dump),
        // then P x V on MFMA (16x16x16, K = the 16 tokens).  Expansion lane:
        // patch 32 half + (lane & 31), tokens 8 (lane >> 5) .. + 7.
#pragma unroll
        for (int hv = 0; hv < 2; hv++) {
            const int pl = lane & 31;
            const int p = 32 * hv + pl;
            const int vgrp = p >> 3, vsub = p & 7;
            const int vbit = 12 * vsub;
            const int vw0 = vgrp * 3 + (vbit >> 5);
            const int vsh = vbit & 31;
            const int vhw = 24 + hv, vhb = pl;
            const _Float16 c3a = hv ? c3v0b : c3v0a, c3b = hv ? c3v1b : c3v1a;
#pragma unroll
            for (int quad = 0; quad < 2; quad++) {
                h4 col[5];
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int tok = 8 * (lane >> 5) + 4 * quad + tt;
                    const uint32_t* vr = &S.vpay[tok * VPAY_TS + w * 26];
                    const uint32_t fld = __builtin_amdgcn_alignbit(vr[vw0 + 1], vr[vw0], vsh) & 0xFFFu;
                    const uint32_t code = (fld & 0x7Fu) | (__builtin_amdgcn_ubfe(vr[vhw], vhb, 1) << 7);
                    const _Float16* ce = &S.cb[p * CB_PS + code * 3];
                    col[0][tt] = ce[0];
                    col[1][tt] = ce[1];
                    col[2][tt] = ce[2];
                    col[3][tt] = ((fld >> 7) & 1u) ? c3b : c3a;
                    col[4][tt] = (_Float16)(unsigned short)((fld >> 8) & 0xFu);
                }
                const int t0 = 8 * (lane >> 5) + 4 * quad;
                *reinterpret_cast<h4*>(&vt[(3 * pl + 0) * VT_CS + t0]) = col[0];
                *reinterpret_cast<h4*>(&vt[(3 * pl + 1) * VT_CS + t0]) = col[1];
                *reinterpret_cast<h4*>(&vt[(3 * pl + 2) * VT_CS + t0]) = col[2];
                *reinterpret_cast<h4*>(&vt[(96 + pl) * VT_CS + t0]) = col[3];
                *reinterpret_cast<h4*>(&vt[(128 + pl) * VT_CS + t0]) = col[4];
            }
            wave_sync();
#pragma unroll
            for (int n = 0; n < 10; n++) {
                const h4 bv = *reinterpret_cast<const h4*>(&vt[(16 * n + li) * VT_CS + 4 * lg]);
                pv[10 * hv + n] = mfma16(Ap[n < 6 ? 0 : (n < 8 ? 1 : 2)], bv, pv[10 * hv + n]);
            }
            wave_sync();
        }

        PHASE(7);
        // ---- (l) advance RoPE base by 16 tokens, stage the next tile
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float sc16 = S.rope[lg][1][u], ss16 = S.rope[lg][2][u];
            const float nc = fmaf(bc[u], sc16, -(bs[u] * ss16));
            const float ns = fmaf(bs[u], sc16, bc[u] * ss16);
            bc[u] = nc;
            bs[u] = ns;
        }
        __syncthreads();
        if (t + 1 < n_tiles) KHQ_COMMIT();
        __syncthreads();
        PHASE(8);
    }

    PHASE(9);
    // ------------------------------------------------ epilogue
    // sums over the 16 tokens (lanes) of each head group
#pragma unroll
    for (int x = 0; x < 2; x++) {
        lsum[x] = row16_sum(lsum[x]);
        s3sum[x] = row16_sum(s3sum[x]);
    }
    float* ep = S.w[w].f;  // [6][256] rotated-domain accumulators
    if (lg < 3) {
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const int h = 2 * lg + x;
#pragma unroll
            for (int hv = 0; hv < 2; hv++) {
#pragma unroll
                for (int n = 0; n < 6; n++) {
                    const int col = 16 * n + li;  // 3 p' + k
                    const int p = 32 * hv + col / 3;
                    ep[h * 256 + 4 * p + col % 3] = pv[10 * hv + n][2 * x] + pv[10 * hv + n][2 * x + 1];
                }
#pragma unroll
                for (int n = 6; n < 8; n++) {
                    const int p = 32 * hv + 16 * (n - 6) + li;
                    const float d3 = pv[10 * hv + n][2 * x] + pv[10 * hv + n][2 * x + 1];
                    const float du = pv[10 * hv + n + 2][2 * x] + pv[10 * hv + n + 2][2 * x + 1];
                    ep[h * 256 + 4 * p + 3] = d3 + du - 8.0f * s3sum[x];
                }
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
        return v > 0 ? v : 255;  // one CU left for the window block
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

#ifdef KHQ_PHASE_TIMING
extern "C" int khq_phase_cycles(unsigned long long* out, int reset) {
    hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(khq::mf::phase_cycles),
                                       sizeof(unsigned long long) * 16);
    if (e == hipSuccess && reset) {
        unsigned long long z[16] = {0};
        e = hipMemcpyToSymbol(HIP_SYMBOL(khq::mf::phase_cycles), z, sizeof(z));
    }
    return e == hipSuccess ? 0 : (int)e;
}
#endif
