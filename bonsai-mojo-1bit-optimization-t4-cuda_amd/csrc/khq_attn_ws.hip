// khq_attn_ws.hip -- compressed-region KHQ attention on MI355X matrix cores,
// wavefront-specialised.
//
// Shape: H_kv = 4 KV heads, 6 query heads per KV head, D = 256, one query
// token.  One 512-thread block per token chunk, tiles of 16 tokens:
//   key wavefronts   0..3 (KV head w): outliers and scores of tile t;
//   value wavefronts 4..7 (KV head w-4): softmax, V decode and P x V of
//                    tile t - 1.
// Each SIMD holds one key and one value wavefront, so one hides the other's
// latency.  The two roles of a KV head hand over through LDS counters (no
// block barrier per tile): the key side publishes a tile's raw scores in a
// double-buffered LDS slot, the value side keeps the running maximum and
// sum and reports when it has read the slot.
//
// The decoded key of row s is   k_s = a_k * norm_s * mult_s * M b_s   with
//   b_s[i] = sgn_i * cb_i                    for codes 0..2 (sgn 0, -1, +1)
//   b_s[i] = sgn_i * (cb_i + res_i * rs_s / mult_s)   for code 3 (outlier)
//   M      = diag(1/(256 d)) * H_256 * blockdiag(R_p)    (fixed per layer)
// and RoPE touches only dims 0..63.  The score splits into
//   pass part:  t . b,  t = R^T H (q[64:] / (256 d)) (query side, fp16 hi+lo);
//   roped part: z = W b (the four 64-blocks of R b summed, exact fp16 rotor
//               entries), then H_64 z (z split hi + lo), RoPE in registers,
//               and the dot with q (key split hi + lo), all on MFMA.
// K contraction order: K-step st, lane group lg, element e <-> dim
// 64 lg + 8 st + e, so lane (token li, lg) owns dims 64 lg .. 64 lg + 63 of
// its token in every K-step.  Outliers are expanded without a walk: per
// tile, each token's outlier payload becomes a rank-window array E[r] =
// (h_r, h_r+1) of fp16 halves h_r = -+nib_r * 2^-24 (sign from the stored
// sign bit; an exact subnormal), so the four halves from any rank r are the
// read pair E[r], E[r + 2].  Per 4-dim group (one mask byte) a table gives
// the sign halves of its codes and the byte selectors that put the window
// halves of its outliers (ranks r .. r + 3, r = outliers before the group)
// at their dims.  The B operand splits into
//   b1 = sgn * cb (an outlier's sign OR-ed in from its window half), exact;
//   b2 = -+nib * 2^-24 at outliers, 0 elsewhere, exact;
// both go through the same A operands and b2's products are scaled by
// 2^24 rs / mult afterwards, per token.
// V is accumulated in the rotated domain; lane (patch 16 g + li, tokens
// 4 lg .. 4 lg + 3) decodes straight into the B operand of 16x16x16 MFMAs:
//   dims (p, k<3): codebook value * (w * a_v * norm * energy)
//   dim  (p, 3):   cents[d3] * (w * a_v * norm) + dump * (w * norm * smeta / 7)
//                  - 8 * sum(w * norm * smeta / 7)
// with the weights split hi + lo.  The inverse V rotor + FWHT + 1/(16 d_v)
// run once per chunk.  Softmax uses a per-head reference maximum that is only
// raised when a tile exceeds it by more than 8 (weights stay <= e^8).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <math.h>
#include <string.h>
#include <stdlib.h>

#include "khq_internal.h"
#include "khq_mfma_util.h"

namespace khq {
namespace ws {

using namespace mu;

#ifdef KHQ_PHASE_TIMING
__device__ unsigned long long phase_cycles[32];
__device__ unsigned long long block_times[1024][2];
#define PHASE(k)                                                              \
    do {                                                                      \
        const unsigned long long now_ = __builtin_amdgcn_s_memtime();         \
        ph_acc[k] += (unsigned)(now_ - ph_t);                                 \
        ph_t = now_;                                                          \
    } while (0)
// wait for the outstanding global loads, then close phase k
#define PHASE_VM(k)                                                           \
    do {                                                                      \
        __builtin_amdgcn_s_waitcnt(0x0F70);                                   \
        PHASE(k);                                                             \
    } while (0)
#define PH_PARAMS , unsigned long long ph_t, unsigned (&ph_acc)[32]
#define PH_ARGS , ph_t, ph_acc
#else
#define PHASE(k) do { } while (0)
#define PHASE_VM(k) do { } while (0)
#define PH_PARAMS
#define PH_ARGS
#endif

constexpr int TT = 16;          // tokens per tile
constexpr int NTHR = 512;       // 4 key + 4 value wavefronts
constexpr int CB_PS = 768;      // halves per codebook patch (256 codes x 3)
constexpr int KP_TS = 12;       // words per staged kpay row: the 40-byte row, 2 zero words
constexpr int KE_S = 68;        // words per token of the rank-window array (ranks 0..67)
constexpr int KE_MAXQ = 50;     // ordinals >= 50 carry no payload (nibble 0, sign -1)
constexpr int VP_TS = 26;       // words per staged vpay row
constexpr float RESCALE_GAP = 8.0f;

struct __align__(16) Smem {
    _Float16 cb[64 * CB_PS];     // V codebook, [patch][code][3]       98304 B
    float o[4][6 * 256];         // setup: query transforms; end: V sums 24576 B
    uint32_t vp[4][TT * VP_TS];  // staged vpay rows per KV head         6656 B
                                 // (setup: rotor_k)
    uint32_t kp[4][TT * KP_TS];  // staged kpay rows per KV head         3072 B
    uint32_t ke[4][TT * KE_S];   // rank windows E[r] = (h_r, h_r+1)    17408 B
    uint4 ktab[256];             // mask byte -> sign halves, window selectors
    uint2 sgb[256];              // 8 flags -> bytes 0x80 / 0 (flags 0..3, 4..7)
    _Float16 cbk[256];           // cents_k[2]
    float pw[2][4][6][TT];       // scaled scores, by tile parity
    float rope[4][3][8];         // per lane group: freq, cos(16 f), sin(16 f)
    _Float16 rotv[64 * 16];      // rotor_v
    _Float16 dvh[256];           // d_v
    _Float16 c3v[2][64];         // cents_v[c][4 p + 3]
    float ml[4][6][2];           // final (max, sum) per query head
    float s3[4][8];              // final dump-offset sums per query head
    int kdone[4];                // tiles whose scores the key wavefront has published
    int vread[4];                // tiles whose scores the value wavefront has read
    int fault;                   // a hand-off wait gave up
};

// Hand-off between the key and value wavefronts of one KV head through LDS
// counters (release / acquire at workgroup scope), so each pair runs at its
// own pace instead of meeting the other pairs at a block barrier every tile.
// The wait is bounded (spin_limit sleeps, 2^20 by default): a wavefront that
// gives up records the fault in the block's LDS flag, and the block then
// writes NaN maxima into its partials and raises the library's device fault
// word (khq_fault_status), so a timed-out result is never silently wrong.
__device__ int g_fault;

__device__ __forceinline__ void wait_count(const int* f, int target, int limit, int* fault) {
    int n = 0;
    while (__hip_atomic_load(f, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if (++n > limit) {
            __hip_atomic_store(fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}
__device__ __forceinline__ void publish_count(int* f, int v) {
    __hip_atomic_store(f, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Loads / stores through global-memory pointers (the batched kernel reads its
// pointers from memory, where the compiler cannot tell their address space
// and would otherwise use flat accesses).
template <typename T>
__device__ __forceinline__ T ldg(const void* p) {
    if constexpr (sizeof(T) % 4 == 0) {
        typedef uint32_t wv __attribute__((ext_vector_type(sizeof(T) / 4)));
        return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) wv*)p);
    } else {
        static_assert(sizeof(T) == 2, "2-byte or word-multiple types");
        return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) unsigned short*)p);
    }
}
template <typename T>
__device__ __forceinline__ void stg(void* p, T v) {
    static_assert(sizeof(T) % 4 == 0, "word-multiple types");
    typedef uint32_t wv __attribute__((ext_vector_type(sizeof(T) / 4)));
    *(__attribute__((address_space(1))) wv*)p = __builtin_bit_cast(wv, v);
}

// Per-lane global inputs of the block set-up, all loaded at kernel entry so
// their latency overlaps the table copies.
struct SetupIn {
    uint2 qr[3];    // q dims 4 lane .. + 3 of the 3 heads this wavefront transforms
    uint2 dkr;      // d_k dims 4 lane .. + 3
    uint4 rk[2];    // rotor_k of patch `lane`
    uint2 qv[4];    // key wavefronts: q dims 16 T' + 4 lg .. + 3 of head min(li / 2, 5)
    unsigned short dj[4];  // key wavefronts: d_k[16 T' + li]
};

__device__ __forceinline__ void load_setup(const AttnArgs& a, int h, int wv, int lane, SetupIn& in) {
    const int li = lane & 15, lg = lane >> 4;
    const __half* qbase = a.q + (size_t)(h * 6 + 3 * (wv >> 2)) * 512;
#pragma unroll
    for (int hd = 0; hd < 3; hd++) in.qr[hd] = ldg<uint2>(qbase + hd * 512 + lane * 4);
    in.dkr = ldg<uint2>(a.dk + lane * 4);
    const uint4* rp = reinterpret_cast<const uint4*>(a.rotor_k + lane * 16);
    in.rk[0] = ldg<uint4>(rp);
    in.rk[1] = ldg<uint4>(rp + 1);
    const __half* qrow = a.q + (size_t)(h * 6 + min(li >> 1, 5)) * 512;
#pragma unroll
    for (int Tp = 0; Tp < 4; Tp++) {
        in.dj[Tp] = ldg<unsigned short>(a.dk + 16 * Tp + li);
        in.qv[Tp] = ldg<uint2>(qrow + 16 * Tp + 4 * lg);
    }
}

// Block-shared constants copied to LDS: loaded at kernel entry, stored
// after the query transforms, so the load latency overlaps that work.
struct TabIn {
    unsigned short cbk, c3;  // cents_k[2][tid] (tid < 256), cents_v[c][4 p + 3] (tid < 128)
    uint4 rot;               // rotor_k (tid 256..383) or rotor_v (tid 384..511), 16 B each
    uint4 dv;                // d_v (tid < 32)
    float rope;              // RoPE table entry tid - 416 (tid >= 416)
};

__device__ __forceinline__ void load_tables(const AttnArgs& a, int tid, TabIn& tb) {
    // unconditional loads (clamped indices): a load under a branch makes the
    // compiler wait for every outstanding load at the join
    const uint4* rsrc = tid < 384 ? reinterpret_cast<const uint4*>(a.rotor_k) + (tid & 127)
                                  : reinterpret_cast<const uint4*>(a.rotor_v) + (tid - 384);
    tb.rot = ldg<uint4>(rsrc);
    tb.cbk = ldg<unsigned short>(a.cents_k + 512 + (tid & 255));
    tb.c3 = ldg<unsigned short>(a.cents_v + ((tid >> 6) & 1) * 256 + (tid & 63) * 4 + 3);
    tb.dv = ldg<uint4>(reinterpret_cast<const uint4*>(a.dv) + (tid & 31));
    tb.rope = ldg<float>(&a.rope_tab[(tid + 64) % 96]);  // entry tid - 416 for tid >= 416
}

__device__ __forceinline__ void store_tables(Smem& S, int tid, const TabIn& tb) {
    if (tid < 256) {
        S.cbk[tid] = __builtin_bit_cast(_Float16, tb.cbk);
    } else if (tid < 384) {
        reinterpret_cast<uint4*>(&S.vp[0][0])[tid - 256] = tb.rot;
    } else {
        reinterpret_cast<uint4*>(S.rotv)[tid - 384] = tb.rot;
    }
    if (tid < 128) S.c3v[tid >> 6][tid & 63] = __builtin_bit_cast(_Float16, tb.c3);
    if (tid < 32) reinterpret_cast<uint4*>(S.dvh)[tid] = tb.dv;
    if (tid >= 416) (&S.rope[0][0][0])[tid - 416] = tb.rope;
}

// Query side of the pass part for 3 query heads of KV head h (heads hd0 ..
// hd0 + 2): tq_hd = R^T H (q_hd[64:] / (256 d)) into S.o[h] as floats [6][256].
__device__ __forceinline__ void query_transform(const SetupIn& in, Smem& S, int h, int hd0,
                                                int lane) {
    float* tq = S.o[h] + hd0 * 256;
    const h4 dk4 = __builtin_bit_cast(h4, in.dkr);
    float dks[4];
#pragma unroll
    for (int c = 0; c < 4; c++) dks[c] = (1.0f / 256.0f) / ((float)dk4[c] + 1e-8f);
    float rk[16];
    {
        const h8 r0 = __builtin_bit_cast(h8, in.rk[0]), r1 = __builtin_bit_cast(h8, in.rk[1]);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            rk[t] = (float)r0[t];
            rk[8 + t] = (float)r1[t];
        }
    }
#pragma unroll
    for (int hd = 0; hd < 3; hd++) {
        const h4 qh = __builtin_bit_cast(h4, in.qr[hd]);
        float u[4];
#pragma unroll
        for (int c = 0; c < 4; c++) u[c] = lane >= 16 ? (float)qh[c] * dks[c] : 0.0f;
        fwht256(u, lane);
        // per patch: t[4p + k] = sum_c u[4p + c] R_p[c][k]
        f4 t;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float x = u[0] * rk[0 * 4 + k];
            x = fmaf(u[1], rk[1 * 4 + k], x);
            x = fmaf(u[2], rk[2 * 4 + k], x);
            x = fmaf(u[3], rk[3 * 4 + k], x);
            t[k] = x;
        }
        *reinterpret_cast<f4*>(&tq[hd * 256 + lane * 4]) = t;
    }
}

// ---------------------------------------------------------------- key role
__device__ __forceinline__ void key_role(const AttnArgs& a, Smem& S, const SetupIn& in,
                                         const TabIn& tb, int h, int lane, int s_lo, int s_hi,
                                         int n_tiles PH_PARAMS) {
    const int li = lane & 15, lg = lane >> 4;
    const float* tq = S.o[h];  // [6][256] query transforms

    // A operands (rows: 2 hd = hi, 2 hd + 1 = lo of head hd; rows 12..15 zero)
    const int arow_h = li >> 1;
    const bool arow_lo = (li & 1) != 0;
    const bool arow_ok = li < 12;
    // signs of 1/d for the H_64 output rows j = 16 T' + li held by this lane's
    // A rows, and q_rot (roped dims 0..63 at the K positions of the rope'd key
    // layout); unconditional loads from a clamped head row, zeroed rows after
    float dsgn[4];
    h8 Aq[2];
    {
        const uint2* qv = in.qv;
#pragma unroll
        for (int Tp = 0; Tp < 4; Tp++)
            dsgn[Tp] = (__half2float(__ushort_as_half(in.dj[Tp])) < 0.0f) ? -1.0f : 1.0f;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const h4 qa = __builtin_bit_cast(h4, qv[2 * kk]), qb = __builtin_bit_cast(h4, qv[2 * kk + 1]);
            const float mq = arow_lo ? -1.0f : 0.0f;
            const uint4 w = uint4{part_pk((float)qa[0], (float)qa[1], mq), part_pk((float)qa[2], (float)qa[3], mq),
                                  part_pk((float)qb[0], (float)qb[1], mq), part_pk((float)qb[2], (float)qb[3], mq)};
            Aq[kk] = __builtin_bit_cast(h8, arow_ok ? w : uint4{0u, 0u, 0u, 0u});
        }
    }
    // ---- staging: mask words 4 lg .. 4 lg + 3 of (token li, head h) straight
    // to registers; kpay rows through LDS; norms to registers.  Buffer loads
    // with a per-lane offset and the tile offset in a scalar register; rows
    // past c_len read as zeros, rows of the next chunk are dropped on commit.
    const int kp_tok0 = lane / 5, kp_part0 = lane % 5;
    const int kp_tok1 = min(lane + 64, 79) / 5, kp_part1 = min(lane + 64, 79) % 5;
    const uint32_t n_rows = (uint32_t)a.c_len * 4;
    const rsrc_t rs_mask = make_rsrc(a.kmask, n_rows * 64);
    const rsrc_t rs_kn = make_rsrc(a.knorm, n_rows * 2);
    const rsrc_t rs_kr = make_rsrc(a.krn, n_rows * 2);
    const rsrc_t rs_kp = make_rsrc(a.kpay, n_rows * 40);
    const uint32_t vo_mask = (uint32_t)(li * 4 + h) * 64 + lg * 16;
    const uint32_t vo_norm = (uint32_t)(li * 4 + h) * 2;
    const uint32_t vo_kp0 = (uint32_t)(kp_tok0 * 4 + h) * 40 + kp_part0 * 8;
    const uint32_t vo_kp1 = (uint32_t)(kp_tok1 * 4 + h) * 40 + kp_part1 * 8;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    u4v m_nx = u4v{0, 0, 0, 0};
    u2v kp_nx0 = u2v{0, 0}, kp_nx1 = u2v{0, 0};
    unsigned short nk_nx = 0, rs_nx = 0;
    auto prefetch = [&](int s0) {
        const int so = s0 * 4;  // first row of the tile
        m_nx = __builtin_amdgcn_raw_buffer_load_b128(rs_mask, vo_mask, so * 64, 0);
        nk_nx = __builtin_amdgcn_raw_buffer_load_b16(rs_kn, vo_norm, so * 2, 0);
        rs_nx = __builtin_amdgcn_raw_buffer_load_b16(rs_kr, vo_norm, so * 2, 0);
        kp_nx0 = __builtin_amdgcn_raw_buffer_load_b64(rs_kp, vo_kp0, so * 40, 0);
        kp_nx1 = __builtin_amdgcn_raw_buffer_load_b64(rs_kp, vo_kp1, so * 40, 0);
    };
    PHASE(16);
    if (n_tiles > 0) prefetch(s_lo);
    query_transform(in, S, h, 0, lane);
    PHASE(27);
    store_tables(S, threadIdx.x, tb);
    PHASE(17);

    __syncthreads();  // (1) tables, staged rotors and query transforms in place
    PHASE(18);

    const float m_lo = arow_lo ? -1.0f : 0.0f;  // part_pk: lo rows take the remainder
    h8 At[8];
#pragma unroll
    for (int st = 0; st < 8; st++) {
        f4 u0 = f4{0.f, 0.f, 0.f, 0.f}, u1 = u0;
        if (arow_ok) {
            u0 = *reinterpret_cast<const f4*>(&tq[arow_h * 256 + 64 * lg + 8 * st]);
            u1 = *reinterpret_cast<const f4*>(&tq[arow_h * 256 + 64 * lg + 8 * st + 4]);
        }
        At[st] = __builtin_bit_cast(h8, uint4{part_pk(u0[0], u0[1], m_lo), part_pk(u0[2], u0[3], m_lo),
                                              part_pk(u1[0], u1[1], m_lo), part_pk(u1[2], u1[3], m_lo)});
    }
    // fold: z_(4q+c') = sum over blocks b of sum_k R_(16b+q)[c'][k] b_(64b+4q+k).
    // K-step st carries q = 2 st + e/4 of block lg; M-tile T = st / 2 holds
    // z rows of q = 4T .. 4T + 3, so the lane row li takes part in K-step st
    // only when li / 8 == st % 2 (s_fold) and then only for e / 4 == (li / 4) % 2.
    const _Float16* rk_lds = reinterpret_cast<const _Float16*>(S.vp);
    const int s_fold = li >> 3;
    h8 Aw[4];
    {
        const bool upper = ((li >> 2) & 1) != 0;  // entries e = 4..7 (else 0..3)
#pragma unroll
        for (int T = 0; T < 4; T++) {
            const int p = 16 * lg + 4 * T + (li >> 2);
            const uint2 r = *reinterpret_cast<const uint2*>(&rk_lds[p * 16 + (li & 3) * 4]);
            Aw[T] = __builtin_bit_cast(h8, upper ? uint4{0u, 0u, r.x, r.y} : uint4{r.x, r.y, 0u, 0u});
        }
    }
    const h8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
    // H_64 = H_4 (x) H_16 (j = 16 T' + li, m = 16 T + 4 lg + c'):
    // A[T'][kk] = sgn(d_j) H_4[T'][2 kk + e/4] H_16[li][4 lg + (e & 3)] / 256;
    // H_4 rows: T'=0 [+ + + +], 1 [+ - + -], 2 [+ + - -], 3 [+ - - +] over
    // T = (kk, e/4).
    h8 Ah[4][2];
    {
        float g4[4];
#pragma unroll
        for (int c = 0; c < 4; c++)
            g4[c] = ((__popc(li & (4 * lg + c)) & 1) ? -1.0f : 1.0f) / 256.0f;
#pragma unroll
        for (int Tp = 0; Tp < 4; Tp++) {
            _Float16 pos[4], neg[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                pos[c] = (_Float16)(g4[c] * dsgn[Tp]);
                neg[c] = -pos[c];
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int T0 = e >> 2, T1 = 2 + (e >> 2);
                Ah[Tp][0][e] = (__popc(Tp & T0) & 1) ? neg[e & 3] : pos[e & 3];
                Ah[Tp][1][e] = (__popc(Tp & T1) & 1) ? neg[e & 3] : pos[e & 3];
            }
        }
    }

    float bc[8], bs[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        bc[u] = 1.0f;
        bs[u] = 0.0f;
    }
    const _Float16* cbq = &S.cbk[64 * lg];
    uint32_t* kpw = S.kp[h];
    uint32_t* kew = S.ke[h];
    // Staged kpay row of a token: the 40 bytes as stored (word 0 c_base_mult,
    // bytes 4..28 nibbles of ordinals 0..49, bytes 29..35 their sign bits),
    // then two zero words.
    // Past the row: word 10 holds nibble word 7 with only ordinals 48, 49
    // (the sign bytes that follow cleared) and word 9 (shared meta) and the
    // sign bits past 49 read as 0, so every rank-window item reads clean
    // words at fixed offsets.
    auto stage_kp = [&](int tok, int part, u2v v) {
        uint32_t* row = &kpw[tok * KP_TS];
        if (part == 4) v = u2v{v[0] & 0x03FFFFFFu, 0u};
        *reinterpret_cast<u2v*>(&row[2 * part]) = v;
        if (part == 3) row[10] = v[1] & 0xFFu;
    };
    // Rank windows: h_r = fp16 bits (sign_r negative ? 0x8000 : 0) | nib_r,
    // i.e. -+nib_r * 2^-24 as an fp16 subnormal (exact; 0x8000 = -0 past
    // ordinal 49, the format's default of residual 0, sign -1), and
    // E[r] = h_r | h_(r+1) << 16 for every rank r, so the four halves from
    // any rank are one read pair E[r], E[r + 2].  Item (token, j) of this
    // lane builds E[8 j .. 8 j + 7] from nibble word 1 + j and sign bits
    // 8 j .. 8 j + 8 (byte 29 + j); E[56 ..] is constant (set up once).
    const int e_it0 = lane, e_it1 = min(lane + 64, 111);
    const bool e_two = lane + 64 < 112;
    auto build_e = [&](int item) {
        const int row = item / 7, j = item - 7 * (item / 7);
        const uint32_t* W = &kpw[row * KP_TS];
        const int sb_w = (29 + j) >> 2, sb_sh = 8 * ((29 + j) & 3);
        const uint32_t nw = W[j < 6 ? 1 + j : 10];        // ordinals 8 j .. 8 j + 7
        const uint32_t nn = W[j < 6 ? 2 + j : 11] & 0xFu;  // ordinal 8 j + 8
        const uint32_t sb = __builtin_amdgcn_alignbit(W[sb_w + 1], W[sb_w], sb_sh);
        const uint2 sg = S.sgb[~sb & 0xFFu];  // negative flags -> byte top bits
        const uint32_t lo = nw & 0x0F0F0F0Fu, hi = (nw >> 4) & 0x0F0F0F0Fu;
        const uint32_t nb01 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // ordinals 0..3
        const uint32_t nb23 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // ordinals 4..7
        const uint32_t H0 = __builtin_amdgcn_perm(sg.x, nb01, 0x05010400u);
        const uint32_t H1 = __builtin_amdgcn_perm(sg.x, nb01, 0x07030602u);
        const uint32_t H2 = __builtin_amdgcn_perm(sg.y, nb23, 0x05010400u);
        const uint32_t H3 = __builtin_amdgcn_perm(sg.y, nb23, 0x07030602u);
        const uint32_t H4 = nn | ((~sb & 0x100u) << 7);
        uint4* dst = reinterpret_cast<uint4*>(&kew[row * KE_S + 8 * j]);
        dst[0] = uint4{H0, __builtin_amdgcn_alignbit(H1, H0, 16), H1, __builtin_amdgcn_alignbit(H2, H1, 16)};
        dst[1] = uint4{H2, __builtin_amdgcn_alignbit(H3, H2, 16), H3, __builtin_amdgcn_alignbit(H4, H3, 16)};
    };
    const uint32_t* kerow = &kew[li * KE_S];
    PHASE(1);

    for (int it = 0; it <= n_tiles; it++) {
        if (it < n_tiles) {
            PHASE_VM(7);
            const int t = it;
            const int s0 = s_lo + t * TT;
            // ---- take the staged tile, start loading the next one
            const bool ok = s0 + li < s_hi;
            const uint4 mc = ok ? uint4{m_nx[0], m_nx[1], m_nx[2], m_nx[3]} : uint4{0, 0, 0, 0};
            const float nk = ok ? __half2float(__ushort_as_half(nk_nx)) : 0.0f;
            const float rs = ok ? __half2float(__ushort_as_half(rs_nx)) : 0.0f;
            stage_kp(kp_tok0, kp_part0, s0 + kp_tok0 < s_hi ? kp_nx0 : u2v{0, 0});
            if (lane < 16) stage_kp(kp_tok1, kp_part1, s0 + kp_tok1 < s_hi ? kp_nx1 : u2v{0, 0});
            if (t + 1 < n_tiles) prefetch(s0 + TT);
            if ((t & 15) == 0) {
#pragma unroll
                for (int u = 0; u < 8; u++)
                    sincos_rev((float)(a.start_pos + s0 + li) * S.rope[lg][0][u], bc[u], bs[u]);
            }
            wave_sync();
            build_e(e_it0);
            if (e_two) build_e(e_it1);
            wave_sync();
            PHASE(2);

            // ---- per-token scalars of this lane's token
            // c_base_mult = word / 1000 when that lies in [0.1, 10] (word in
            // [100, 10000]), else 1; the product with the rounded 1 / 1000
            // and the hardware reciprocal are within 2 ulp of the quotients
            const uint32_t mraw = kpw[li * KP_TS];
            const bool m_ok = mraw - 100u <= 9900u;
            const float mult = m_ok ? (float)mraw * 0.001f : 1.0f;
            const float rr = rs * __builtin_amdgcn_rcpf(mult);
            const float fsc = a.a_k * nk * mult * a.sc;

            // ---- outliers (code 3) of dims 64 lg .. 64 lg + 63: flags at the
            // even bit of each code, and the rank of the first one (outliers
            // of the quarters before this lane's)
            const uint32_t mw[4] = {mc.x, mc.y, mc.z, mc.w};
            uint32_t ow[4];
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ow[i] = (mw[i] & (mw[i] >> 1)) & 0x55555555u;
                cnt += __popc(ow[i]);
            }
            int qrun;
            {
                // outliers of the quarters before this lane's, across the 4 lane
                // rows of the token (row swaps, no LDS round trip)
                const auto p16 = __builtin_amdgcn_permlane16_swap((uint32_t)cnt, (uint32_t)cnt, false, false);
                const uint32_t c_even = p16[0], c_odd = p16[1];  // rows 2 k, 2 k + 1
                const uint32_t pair = c_even + c_odd;
                const auto p32 = __builtin_amdgcn_permlane32_swap(pair, pair, false, false);
                qrun = (int)(((lg & 1) ? c_even : 0u) + ((lg >= 2) ? p32[0] : 0u));
            }

            PHASE(3);
            // ---- b1 / b2 operands + pass / fold MFMAs.  Per 4-dim group (a
            // mask byte): the table gives the sign halves (codes 1 / 2 / 3 ->
            // -1 / +1 / +1) and the selectors that place the window halves of
            // the group's outliers at their dims; the outlier's own sign then
            // comes from its window half (b1 = sign * cb, b2 = -+nib * 2^-24).
            f4 cs = f4{0.f, 0.f, 0.f, 0.f}, cs2 = cs;
            f4 zt[4], zt2[4];
#pragma unroll
            for (int T = 0; T < 4; T++) {
                zt[T] = f4{0.f, 0.f, 0.f, 0.f};
                zt2[T] = zt[T];
            }
            {
                int q = 0;
#pragma unroll
                for (int st = 0; st < 8; st++) {
                    const uint32_t word = mw[st >> 1], owd = ow[st >> 1];
                    const int sh = 16 * (st & 1);
                    // ranks past 49 all read the constant window: the rank is
                    // clamped once per mask word (at most 16 more before the
                    // next clamp, so every read stays inside the token's row)
                    if ((st & 1) == 0) q = min(qrun, KE_MAXQ);
                    const int rA = q;
                    const int rB = rA + __popc(__builtin_amdgcn_ubfe(owd, sh, 8));
                    q = rA + __popc(__builtin_amdgcn_ubfe(owd, sh, 16));
                    if (st & 1) qrun = q;
                    const uint4 tA = S.ktab[__builtin_amdgcn_ubfe(word, sh, 8)];
                    const uint4 tB = S.ktab[__builtin_amdgcn_ubfe(word, sh + 8, 8)];
                    const uint32_t eA0 = kerow[rA], eA1 = kerow[rA + 2];
                    const uint32_t eB0 = kerow[rB], eB1 = kerow[rB + 2];
                    const uint32_t nv[4] = {__builtin_amdgcn_perm(eA1, eA0, tA.z),
                                            __builtin_amdgcn_perm(eA1, eA0, tA.w),
                                            __builtin_amdgcn_perm(eB1, eB0, tB.z),
                                            __builtin_amdgcn_perm(eB1, eB0, tB.w)};
                    const uint32_t sgv[4] = {tA.x, tA.y, tB.x, tB.y};
                    const uint4 cbw = *reinterpret_cast<const uint4*>(&cbq[8 * st]);
                    const uint32_t cbv[4] = {cbw.x, cbw.y, cbw.z, cbw.w};
                    uint32_t b1w[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t sg = (nv[k] & 0x80008000u) | sgv[k];
                        b1w[k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, sg) * __builtin_bit_cast(h2, cbv[k]));
                    }
                    const h8 b1 = __builtin_bit_cast(h8, uint4{b1w[0], b1w[1], b1w[2], b1w[3]});
                    const h8 b2 = __builtin_bit_cast(h8, uint4{nv[0], nv[1], nv[2], nv[3]});
                    cs = mfma32(At[st], b1, cs);
                    cs2 = mfma32(At[st], b2, cs2);
                    const h8 aw = (st & 1) == s_fold ? Aw[st >> 1] : hzero;
                    zt[st >> 1] = mfma32(aw, b1, zt[st >> 1]);
                    zt2[st >> 1] = mfma32(aw, b2, zt2[st >> 1]);
                }
                const float rr24 = rr * 16777216.0f;  // b2 carries nib * 2^-24
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    cs[c] = fmaf(rr24, cs2[c], cs[c]);
#pragma unroll
                    for (int T = 0; T < 4; T++) zt[T][c] = fmaf(rr24, zt2[T][c], zt[T][c]);
                }
            }

            PHASE(4);
            // ---- H_64 (1/(256 d)) on z (z rounded to fp16, nearest)
            f4 kr[4];
            {
                h8 zb[2];
#pragma unroll
                for (int k = 0; k < 2; k++)
                    zb[k] = __builtin_bit_cast(
                        h8, uint4{pk_rne(zt[2 * k][0], zt[2 * k][1]), pk_rne(zt[2 * k][2], zt[2 * k][3]),
                                  pk_rne(zt[2 * k + 1][0], zt[2 * k + 1][1]),
                                  pk_rne(zt[2 * k + 1][2], zt[2 * k + 1][3])});
#pragma unroll
                for (int Tp = 0; Tp < 4; Tp++) {
                    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
                    acc = mfma32(Ah[Tp][0], zb[0], acc);
                    acc = mfma32(Ah[Tp][1], zb[1], acc);
                    kr[Tp] = acc;
                }
            }

            // ---- RoPE at absolute position start_pos + s0 + li
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int T0 = u >> 2, cc = u & 3;
                const float x0 = kr[T0][cc], x1 = kr[T0 + 2][cc];
                kr[T0][cc] = fmaf(x0, bc[u], -(x1 * bs[u]));
                kr[T0 + 2][cc] = fmaf(x0, bs[u], x1 * bc[u]);
            }

            // ---- roped part of the score on MFMA (key rounded to fp16, nearest)
            {
                h8 kb[2];
#pragma unroll
                for (int k = 0; k < 2; k++)
                    kb[k] = __builtin_bit_cast(
                        h8, uint4{pk_rne(kr[2 * k][0], kr[2 * k][1]), pk_rne(kr[2 * k][2], kr[2 * k][3]),
                                  pk_rne(kr[2 * k + 1][0], kr[2 * k + 1][1]),
                                  pk_rne(kr[2 * k + 1][2], kr[2 * k + 1][3])});
                cs = mfma32(Aq[0], kb[0], cs);
                cs = mfma32(Aq[1], kb[1], cs);
            }

            // ---- scores of heads 2 lg, 2 lg + 1 for token li
            const bool tok_ok = (s0 + li) < s_hi;
            float sc2[2];
            sc2[0] = tok_ok ? (cs[0] + cs[1]) * fsc : -INFINITY;
            sc2[1] = tok_ok ? (cs[2] + cs[3]) * fsc : -INFINITY;
            if (lg == 3) {
                sc2[0] = -INFINITY;
                sc2[1] = -INFINITY;
            }

            // ---- raw scores to the value side (it keeps the softmax state);
            // buffer t & 1 last held tile t - 2
            const int buf = t & 1;
            PHASE(5);
            wait_count(&S.vread[h], t - 1, a.spin_limit, &S.fault);
            PHASE(23);
            if (lg < 3) {
                S.pw[buf][h][2 * lg][li] = sc2[0];
                S.pw[buf][h][2 * lg + 1][li] = sc2[1];
            }
            publish_count(&S.kdone[h], t + 1);

            // ---- advance the lane's RoPE angles by 16 tokens
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float sc16 = S.rope[lg][1][u], ss16 = S.rope[lg][2][u];
                const float nc = fmaf(bc[u], sc16, -(bs[u] * ss16));
                const float ns = fmaf(bs[u], sc16, bc[u] * ss16);
                bc[u] = nc;
                bs[u] = ns;
            }
        }
        PHASE(5);
        if (it == 0) __syncthreads();  // (2) the value side's codebook copy is complete
        PHASE(6);
    }

    __syncthreads();  // (3) maxima / sums / dump sums published
    __syncthreads();  // (4) V sums in place
    PHASE(21);
}

// -------------------------------------------------------------- value role
__device__ __forceinline__ void value_role(const AttnArgs& a, Smem& S, const SetupIn& in,
                                           const TabIn& tb, int h, int lane, int s_lo, int s_hi,
                                           int n_tiles PH_PARAMS) {
    const int li = lane & 15, lg = lane >> 4;

    const int r_head = li >> 1;       // A row li: head li / 2, hi (even) or lo (odd)
    const bool r_lo = (li & 1) != 0;
    const bool r_ok = li < 12;
    const float m_lo = r_lo ? -1.0f : 0.0f;  // part_pk: lo rows take the remainder

    // staging: vpay rows (13 uint2 per token) by lane, norms of token li
    int vp_tok[4], vp_part[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int idx = min(lane + 64 * k, TT * 13 - 1);
        vp_tok[k] = idx / 13;
        vp_part[k] = idx % 13;
    }
    // Buffer loads: per-lane offsets, tile offset in a scalar register; rows
    // past c_len read as zeros, rows of the next chunk are dropped on commit.
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    const uint32_t n_rows = (uint32_t)a.c_len * 4;
    const rsrc_t rs_vp = make_rsrc(a.vpay, n_rows * 104);
    const rsrc_t rs_vn = make_rsrc(a.vnorm, n_rows * 2);
    const rsrc_t rs_ve = make_rsrc(a.vrn, n_rows * 2);
    const rsrc_t rs_vm = make_rsrc(a.vsm, n_rows * 4);
    uint32_t vo_vp[4];
#pragma unroll
    for (int k = 0; k < 4; k++) vo_vp[k] = (uint32_t)(vp_tok[k] * 4 + h) * 104 + vp_part[k] * 8;
    // norms of token 4 lg + (li & 3): the lane quad holds this lane group's tokens
    const int n_tok = 4 * lg + (li & 3);
    const uint32_t vo_n = (uint32_t)(n_tok * 4 + h);
    u2v vp_nx[4];
    unsigned short vn_nx = 0, ve_nx = 0;
    uint32_t vm_nx = 0;
    auto prefetch = [&](int s0) {
        const int so = s0 * 4;
#pragma unroll
        for (int k = 0; k < 4; k++)
            vp_nx[k] = __builtin_amdgcn_raw_buffer_load_b64(rs_vp, vo_vp[k], so * 104, 0);
        vn_nx = __builtin_amdgcn_raw_buffer_load_b16(rs_vn, vo_n * 2, so * 2, 0);
        ve_nx = __builtin_amdgcn_raw_buffer_load_b16(rs_ve, vo_n * 2, so * 2, 0);
        vm_nx = __builtin_amdgcn_raw_buffer_load_b32(rs_vm, vo_n * 4, so * 4, 0);
    };
    if (n_tiles > 0) prefetch(s_lo);
    query_transform(in, S, h, 3, lane);
    store_tables(S, threadIdx.x, tb);
    PHASE(19);
    __syncthreads();  // (1)
    PHASE(8);
    // V codebook (96 KB), copied by these wavefronts alone while the key
    // wavefronts start on the first tile; it is read from the first decode on,
    // which comes after the next block barrier.
    {
        const int vt = h * 64 + lane;
        const uint4* cbsrc = reinterpret_cast<const uint4*>(a.vq);
        uint4* cbdst = reinterpret_cast<uint4*>(S.cb);
#pragma unroll
        for (int b = 0; b < 2; b++) {
            uint4 cbt[12];
#pragma unroll
            for (int i = 0; i < 12; i++) cbt[i] = ldg<uint4>(cbsrc + vt + 256 * (12 * b + i));
#pragma unroll
            for (int i = 0; i < 12; i++) cbdst[vt + 256 * (12 * b + i)] = cbt[i];
        }
    }
    PHASE(20);
    // lane constants: patch p = 16 g + li for g = 0..3
    // (cents_v[0][4 p + 3], cents_v[1][4 p + 3]) as one packed pair
    uint32_t c3w[4];
#pragma unroll
    for (int g = 0; g < 4; g++)
        c3w[g] = (uint32_t)__builtin_bit_cast(unsigned short, S.c3v[0][16 * g + li]) |
                 ((uint32_t)__builtin_bit_cast(unsigned short, S.c3v[1][16 * g + li]) << 16);

    f4 pv[20];
#pragma unroll
    for (int n = 0; n < 20; n++) pv[n] = f4{0.f, 0.f, 0.f, 0.f};
    float s3p = 0.0f;  // sum of w * norm * smeta / 7 over this lane's tokens (hi rows)
    float Mref = -INFINITY, lsum = 0.0f;  // softmax state of head r_head
    const float av = a.a_v;
    uint32_t* vpw = S.vp[h];
    PHASE(9);

    for (int it = 0; it <= n_tiles; it++) {
        if (it >= 1) {
            PHASE_VM(14);
            const int t = it - 1;
            const int buf = t & 1;
            // ---- the key side's scores of this tile: row head r_head, tokens
            // 4 lg .. 4 lg + 3 (read first: their latency overlaps the staging)
            PHASE(14);
            wait_count(&S.kdone[h], t + 1, a.spin_limit, &S.fault);
            PHASE(22);
            f4 sc4 = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            if (r_ok) sc4 = *reinterpret_cast<const f4*>(&S.pw[buf][h][r_head][4 * lg]);
            // ---- take the staged tile, start loading the next one
            const int s0 = s_lo + t * TT;
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (lane + 64 * k < TT * 13)
                    *reinterpret_cast<u2v*>(&vpw[vp_tok[k] * VP_TS + vp_part[k] * 2]) =
                        s0 + vp_tok[k] < s_hi ? vp_nx[k] : u2v{0, 0};
            PHASE(10);
            // V scalings of token n_tok, then of tokens 4 lg .. 4 lg + 3 from
            // the lane quad (DPP broadcast)
            float sv[3][4];
            {
                const bool ok = s0 + n_tok < s_hi;
                const float nv = ok ? __half2float(__ushort_as_half(vn_nx)) : 0.0f;
                const float en = ok ? __half2float(__ushort_as_half(ve_nx)) : 0.0f;
                const float vm = ok ? __uint_as_float(vm_nx) : 0.0f;
                const float own[3] = {(av * nv) * en, av * nv, nv * vm / 7.0f};
#pragma unroll
                for (int v = 0; v < 3; v++) {
                    sv[v][0] = dpp<0x00>(own[v]);
                    sv[v][1] = dpp<0x55>(own[v]);
                    sv[v][2] = dpp<0xAA>(own[v]);
                    sv[v][3] = dpp<0xFF>(own[v]);
                }
            }
            if (t + 1 < n_tiles) prefetch(s_lo + (t + 1) * TT);
            wave_sync();

            // ---- softmax of head r_head with a lazily raised reference
            // maximum (the same state in every lane of the head)
            float mx = fmaxf(fmaxf(sc4[0], sc4[1]), fmaxf(sc4[2], sc4[3]));
            {
                // across the four lane rows: row-pair and half swaps (VALU)
                const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                                  false, false);
                mx = fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
                const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                                  false, false);
                mx = fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
            }
            const bool need = mx > Mref + RESCALE_GAP;
            if (__ballot(need) != 0ull) {
                const float nm = need ? mx : Mref;
                const float fr = (nm == -INFINITY) ? 1.0f : fexp(Mref - nm);
                Mref = nm;
                lsum *= fr;
                s3p *= fr;
                // C rows 4 lg + c hold heads 2 lg + c / 2: factors from the
                // lanes whose A rows are those heads (lane 16 lg + 4 lg + 2 x)
                const float f0 = lg < 3 ? __shfl(fr, 20 * lg, 64) : 1.0f;
                const float f1 = lg < 3 ? __shfl(fr, 20 * lg + 2, 64) : 1.0f;
#pragma unroll
                for (int n = 0; n < 20; n++) {
                    pv[n][0] *= f0;
                    pv[n][1] *= f0;
                    pv[n][2] *= f1;
                    pv[n][3] *= f1;
                }
            }
            f4 pw4;
#pragma unroll
            for (int c = 0; c < 4; c++) pw4[c] = (sc4[c] == -INFINITY) ? 0.0f : fexp(sc4[c] - Mref);
            lsum += (pw4[0] + pw4[1]) + (pw4[2] + pw4[3]);
            publish_count(&S.vread[h], t + 1);

            // ---- weights x V scalings -> A operands (rows head hi/lo, K = tokens 4 lg..)
            h4 Ap[3];
            {
#pragma unroll
                for (int v = 0; v < 3; v++) {
                    const f4 w = pw4 * f4{sv[v][0], sv[v][1], sv[v][2], sv[v][3]};
                    if (v == 2 && !r_lo) s3p += (w[0] + w[1]) + (w[2] + w[3]);
                    const uint2 pk = uint2{part_pk(w[0], w[1], m_lo), part_pk(w[2], w[3], m_lo)};
                    Ap[v] = __builtin_bit_cast(h4, pk);
                }
            }

            PHASE(11);
            // ---- decode V straight into B operands, P x V on MFMA
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int p = 16 * g + li;
                const int vbit = 12 * (p & 7);
                const int vw0 = (p >> 3) * 3 + (vbit >> 5);
                const int vsh = vbit & 31;
                const int vhw = 24 + (g >> 1), vhb = p & 31;
                h4 b0, b1, b2;
                uint32_t fl[4];
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const uint32_t* vr = &vpw[(4 * lg + tt) * VP_TS];
                    const uint32_t fld = __builtin_amdgcn_alignbit(vr[vw0 + 1], vr[vw0], vsh);
                    fl[tt] = fld;
                    const uint32_t code = (fld & 0x7Fu) | (__builtin_amdgcn_ubfe(vr[vhw], vhb, 1) << 7);
                    const _Float16* ce = &S.cb[p * CB_PS + code * 3];
                    b0[tt] = ce[0];
                    b1[tt] = ce[1];
                    b2[tt] = ce[2];
                }
                // tokens in pairs: the low 16 bits of both fields in one word;
                // bit 7 picks cents_v[bit][4 p + 3] (byte selectors of c3w),
                // bits 8..11 are the nibble (1024 + nib as fp16, minus 1024)
                uint32_t w3[2], w4[2];
#pragma unroll
                for (int pr = 0; pr < 2; pr++) {
                    const uint32_t x = __builtin_amdgcn_perm(fl[2 * pr + 1], fl[2 * pr], 0x05040100u);
                    const uint32_t sel = ((x >> 6) & 0x00020002u) * 0x0101u + 0x01000100u;
                    w3[pr] = __builtin_amdgcn_perm(c3w[g], c3w[g], sel);
                    const h2 n = __builtin_bit_cast(h2, ((x >> 8) & 0x000F000Fu) | 0x64006400u);
                    w4[pr] = __builtin_bit_cast(uint32_t, n - h2{(_Float16)1024.0f, (_Float16)1024.0f});
                }
                const h4 b3 = __builtin_bit_cast(h4, uint2{w3[0], w3[1]});
                const h4 b4 = __builtin_bit_cast(h4, uint2{w4[0], w4[1]});
                pv[5 * g + 0] = mfma16(Ap[0], b0, pv[5 * g + 0]);
                pv[5 * g + 1] = mfma16(Ap[0], b1, pv[5 * g + 1]);
                pv[5 * g + 2] = mfma16(Ap[0], b2, pv[5 * g + 2]);
                pv[5 * g + 3] = mfma16(Ap[1], b3, pv[5 * g + 3]);
                pv[5 * g + 4] = mfma16(Ap[2], b4, pv[5 * g + 4]);
            }
        }
        PHASE(12);
        if (it == 0) __syncthreads();  // (2) codebook copy complete
        PHASE(13);
    }

    // ---- epilogue: dump sums per head (hi rows li = 2 hd, all lane groups)
    s3p += __shfl_xor(s3p, 16, 64);
    s3p += __shfl_xor(s3p, 32, 64);
    lsum += xor_lane<16>(lsum);
    lsum += xor_lane<32>(lsum);
    if (lg == 0 && r_ok && !r_lo) {
        S.s3[h][r_head] = s3p;
        S.ml[h][r_head][0] = Mref;
        S.ml[h][r_head][1] = lsum;
    }
    __syncthreads();  // (3)
    // rotated-domain sums [6][256] in the key strip area of this KV head
    float* ep = S.o[h];
    if (lg < 3) {
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const int hd = 2 * lg + x;
            const float off = 8.0f * S.s3[h][hd];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int p = 16 * g + li;
#pragma unroll
                for (int k = 0; k < 3; k++)
                    ep[hd * 256 + 4 * p + k] = pv[5 * g + k][2 * x] + pv[5 * g + k][2 * x + 1];
                ep[hd * 256 + 4 * p + 3] = (pv[5 * g + 3][2 * x] + pv[5 * g + 3][2 * x + 1]) +
                                           (pv[5 * g + 4][2 * x] + pv[5 * g + 4][2 * x + 1]) - off;
            }
        }
    }
    __syncthreads();  // (4)
    PHASE(21);
}

// ------------------------------------------------------------ window blocks
// The raw ring window (fp16, K already roped) of KV head hk, in one of four
// blocks (one per KV head) after the last compressed chunk, used when the
// launch has CUs to spare; the four write the rows of their 6 query heads
// into the same partial.  Wavefront w takes window rows w hw .. + hw - 1
// (hw = 16 or 32, win_len <= 256); every K and V load of its rows is issued
// at entry, so the block waits for memory once:
//   scores q.k on MFMA (A = the 6 query rows, B = K rows, exact fp16, fp32
//   accumulate) into LDS;
//   softmax per query head over the whole window (wavefront i < 6 takes head i);
//   P x V on the vector ALUs, lane l holding dims 4 l .. 4 l + 3, then the 8
//   wavefronts' numerators are summed through LDS.
constexpr int NWIN = 4;  // window blocks per sequence
__device__ __forceinline__ void window_block(const AttnArgs& a, Smem& S, int part_idx, int hk) {
    constexpr int WMAX = 256;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;
    const int wl = a.win_len;
    const int hw = wl > 128 ? 32 : 16;  // rows per wavefront
    const int r_lo = wv * hw, r_hi = min(wl, r_lo + hw);
    float* sp = reinterpret_cast<float*>(S.cb);  // [6][WMAX] scores, then weights
    float* sml = sp + 6 * WMAX;                  // [6][2] max, sum
    float* sacc = sml + 16;                      // [8][6][256] numerators per wavefront
    auto slot_of = [&](int s) {
        const int x = a.win_start + s;
        return x >= a.ring_cap ? x - a.ring_cap : x;
    };
    // ---- all loads first: q rows, this wavefront's K rows and V rows
    h8 Aqk[8];
    {
        const __half* qrow = a.q + (size_t)(hk * 6 + min(li, 5)) * 512;
#pragma unroll
        for (int st = 0; st < 8; st++) {
            const uint4 v = ldg<uint4>(qrow + 32 * st + 8 * lg);
            Aqk[st] = __builtin_bit_cast(h8, li < 6 ? v : uint4{0u, 0u, 0u, 0u});
        }
    }
    const int last = max(wl - 1, 0);
    // ring rows through buffer loads (32-bit offsets): K rows of both tiles and
    // the V rows of the first 16 at entry, the other 16 V rows (32-row
    // wavefronts) during the scores
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    const uint32_t ring_bytes = (uint32_t)a.ring_cap * a.h_kv * 512;
    const rsrc_t rsk = make_rsrc(a.ring_k, ring_bytes);
    const rsrc_t rsv = make_rsrc(a.ring_v, ring_bytes);
    auto row_off = [&](int s) { return ((uint32_t)slot_of(min(s, last)) * a.h_kv + hk) * 512; };
    u4v kv[2][8];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t o = row_off(r_lo + 16 * u + li) + 16 * lg;
#pragma unroll
        for (int st = 0; st < 8; st++)
            kv[u][st] = (u == 0 || hw == 32) ? __builtin_amdgcn_raw_buffer_load_b128(rsk, o, 64 * st, 0)
                                             : u4v{0u, 0u, 0u, 0u};
    }
    u2v vr[16];
    auto load_v = [&](int base) {
#pragma unroll
        for (int u = 0; u < 16; u++)
            vr[u] = __builtin_amdgcn_raw_buffer_load_b64(rsv, row_off(base + u) + 8 * lane, 0, 0);
    };
    float acc[6][4];
#pragma unroll
    for (int i = 0; i < 6; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[i][c] = 0.0f;
    load_v(r_lo);
    // ---- scores of this wavefront's rows
#pragma unroll
    for (int u = 0; u < 2; u++) {  // the second tile only for 32-row wavefronts
        const int s = r_lo + 16 * u + li;
        f4 sacc4 = f4{0.f, 0.f, 0.f, 0.f};
        if (u == 0 || hw == 32) {
#pragma unroll
            for (int st = 0; st < 8; st++)
                sacc4 = mfma32(Aqk[st], __builtin_bit_cast(h8, kv[u][st]), sacc4);
        }
        // C rows 4 lg + c = query head, column li = row s
        if (lg < 2) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int hd = 4 * lg + c;
                if (hd < 6 && s < r_hi) sp[hd * WMAX + s] = sacc4[c] * a.sc;
            }
        }
    }
    __syncthreads();
    // ---- softmax: wavefront i < 6 owns query head i
    if (wv < 6) {
        float* row = sp + wv * WMAX;
        float m = -INFINITY;
        for (int s = lane; s < wl; s += 64) m = fmaxf(m, row[s]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float l = 0.0f;
        for (int s = lane; s < wl; s += 64) {
            const float p = __expf(row[s] - m);
            row[s] = p;
            l += p;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
        if (lane == 0) {
            sml[wv * 2 + 0] = m;
            sml[wv * 2 + 1] = l;
        }
    }
    __syncthreads();
    // ---- P x V over this wavefront's rows (rows past r_hi weigh 0)
    auto pv16 = [&](int base) {
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const bool ok = base + u < r_hi;
            const int su = min(base + u, WMAX - 1);
            const h4 vh = __builtin_bit_cast(h4, vr[u]);
#pragma unroll
            for (int i = 0; i < 6; i++) {
                const float p = ok ? sp[i * WMAX + su] : 0.0f;
#pragma unroll
                for (int c = 0; c < 4; c++) acc[i][c] = fmaf(p, (float)vh[c], acc[i][c]);
            }
        }
    };
    pv16(r_lo);
    if (hw == 32) {
        load_v(r_lo + 16);
        pv16(r_lo + 16);
    }
#pragma unroll
    for (int i = 0; i < 6; i++)
        *reinterpret_cast<f4*>(&sacc[(wv * 6 + i) * 256 + 4 * lane]) =
            f4{acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
    __syncthreads();
    // ---- sum the 8 wavefronts: thread t takes dims of (head, dim) pairs t, t + 512, t + 1024
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int e = tid + 512 * j;  // e = head * 256 + dim
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < 8; w++) v += sacc[w * 6 * 256 + e];
        const int i = e >> 8, d = e & 255;
        float* out = a.part + ((size_t)(hk * 6 + i) * a.part_stride + part_idx) * 258;
        stg<float>(&out[d], v);
        if (d == 0) {
            stg<float>(&out[256], sml[i * 2 + 0]);
            stg<float>(&out[257], sml[i * 2 + 1]);
        }
    }
}

// The raw ring window (fp16, K already roped) for all 24 query heads in one
// block (used when the chunks leave no CU for one block per KV head: the
// chunks then take several tiles each and hide it).  Wavefront w serves KV head w % 4
// and half w / 4 of the window rows (win_len <= 256):
//   scores q.k on MFMA (A = the 6 query rows of the group, B = K rows, both
//   exact fp16, fp32 accumulate) into LDS;
//   softmax per query head over the whole window in LDS;
//   P x V on the matrix cores (below);
// then the two halves of each KV head are added into one partial triple.
__device__ void window_block_all(const AttnArgs& a, Smem& S, int part_idx) {
    constexpr int WMAX = 256;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;
    const int hk = wv & 3, half = wv >> 2;
    const int wl = a.win_len;
    const int hw = ((wl + 31) / 32) * 16;  // rows per half, a multiple of 16
    const int r_lo = half * hw, r_hi = min(wl, r_lo + hw);
    float* sp = reinterpret_cast<float*>(S.cb);          // [4][6][WMAX] scores, then weights
    float* sml = sp + 4 * 6 * WMAX;                      // [4][6][2] max, sum
    float* sacc = sml + 4 * 6 * 2;                       // [4][6][256] half-1 numerators
    auto slot_of = [&](int s) {
        const int x = a.win_start + s;
        return x >= a.ring_cap ? x - a.ring_cap : x;
    };
    // ---- scores: rows 0..5 of A are the group's query heads (hi only: q is fp16)
    h8 Aqk[8];
    {
        const __half* qrow = a.q + (size_t)(hk * 6 + min(li, 5)) * 512;
#pragma unroll
        for (int st = 0; st < 8; st++) {
            const uint4 v = ldg<uint4>(qrow + 32 * st + 8 * lg);
            Aqk[st] = __builtin_bit_cast(h8, li < 6 ? v : uint4{0u, 0u, 0u, 0u});
        }
    }
    for (int r0 = r_lo; r0 < r_hi; r0 += 32) {  // two 16-row tiles' loads in flight
        uint4 kv[2][8];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int slot = slot_of(min(r0 + 16 * u + li, wl - 1));
            const __half* krow = a.ring_k + ((size_t)slot * a.h_kv + hk) * 256 + 8 * lg;
#pragma unroll
            for (int st = 0; st < 8; st++) kv[u][st] = ldg<uint4>(krow + 32 * st);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int s = r0 + 16 * u + li;
            if (r0 + 16 * u >= r_hi) break;
            f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 8; st++) acc = mfma32(Aqk[st], __builtin_bit_cast(h8, kv[u][st]), acc);
            // C rows 4 lg + c = query head, column li = row s
            if (lg < 2) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int hd = 4 * lg + c;
                    if (hd < 6 && s < r_hi) sp[(hk * 6 + hd) * WMAX + s] = acc[c] * a.sc;
                }
            }
        }
    }
    __syncthreads();
    // ---- softmax: wavefront (hk, half) owns heads 3 half .. + 2 of KV head hk
#pragma unroll
    for (int i = 0; i < 3; i++) {
        float* row = sp + (hk * 6 + 3 * half + i) * WMAX;
        float m = -INFINITY;
        for (int s = lane; s < wl; s += 64) m = fmaxf(m, row[s]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float l = 0.0f;
        for (int s = lane; s < wl; s += 64) {
            const float p = __expf(row[s] - m);
            row[s] = p;
            l += p;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
        if (lane == 0) {
            sml[(hk * 6 + 3 * half + i) * 2 + 0] = m;
            sml[(hk * 6 + 3 * half + i) * 2 + 1] = l;
        }
    }
    __syncthreads();
    // ---- P x V on the matrix cores over this half's rows:
    // O^T [dim][head] = V^T [dim][token] P^T [token][head] with 16x16x16
    // MFMAs (M = 16 dims, N = the 6 query heads, K = 16 tokens); the weights
    // enter as fp16 hi + lo (two MFMAs), V exact.  Each wavefront stages its
    // 16-token V groups transposed in its own LDS region: lane l's dims
    // 4 l .. 4 l + 3 become 4 rows of 16 tokens.  Group g + 1's rows load
    // while group g is used.
    constexpr int VT_LD = 20;  // halves per staged V^T row (16 tokens + pad; 8-byte rows)
    _Float16* vts = reinterpret_cast<_Float16*>(sacc + 4 * 6 * 256) + wv * 256 * VT_LD;
    const int n_g = (r_hi - r_lo + 15) / 16;  // 16-token groups of this half
    auto load_v = [&](uint2 (&vr)[16], int s0) {
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int slot = slot_of(min(s0 + u, r_hi - 1));
            vr[u] = ldg<uint2>(a.ring_v + ((size_t)slot * a.h_kv + hk) * 256 + 4 * lane);
        }
    };
    f4 o[16];
#pragma unroll
    for (int i = 0; i < 16; i++) o[i] = f4{0.f, 0.f, 0.f, 0.f};
    const int n = li, kg = lg;  // B / C column: query head n; K group kg
    auto group = [&](const uint2 (&vr)[16], int s0) {
        // V^T rows 4 lane + c, tokens s0 .. s0 + 15
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            uint32_t wds[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t x0 = (c < 2) ? vr[2 * u].x : vr[2 * u].y;
                const uint32_t x1 = (c < 2) ? vr[2 * u + 1].x : vr[2 * u + 1].y;
                wds[u] = __builtin_amdgcn_perm(x1, x0, sel);
            }
            uint2* row = reinterpret_cast<uint2*>(vts + (4 * lane + c) * VT_LD);
#pragma unroll
            for (int q = 0; q < 4; q++) row[q] = uint2{wds[2 * q], wds[2 * q + 1]};
        }
        // P^T: tokens s0 + 4 kg .. + 3 of head n (rows past r_hi and heads
        // past 5 weigh 0), split hi + lo
        f4 pw = f4{0.f, 0.f, 0.f, 0.f};
        if (n < 6) pw = *reinterpret_cast<const f4*>(&sp[(hk * 6 + n) * WMAX + min(s0 + 4 * kg, WMAX - 4)]);
        h4 bh, bl;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float p = (s0 + 4 * kg + j < r_hi) ? pw[j] : 0.0f;
            const _Float16 h = (_Float16)p;
            bh[j] = h;
            bl[j] = (_Float16)(p - (float)h);
        }
        wave_sync();  // this wavefront's V^T rows are in place
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const h4 av = *reinterpret_cast<const h4*>(vts + (16 * i + n) * VT_LD + 4 * kg);
            o[i] = mfma16(av, bh, o[i]);
            o[i] = mfma16(av, bl, o[i]);
        }
        wave_sync();  // the rows are read before the next group overwrites them
    };
    {
        uint2 vrA[16], vrB[16];
        if (n_g > 0) load_v(vrA, r_lo);
        if (n_g > 1) load_v(vrB, r_lo + 16);
        for (int g = 0; g < n_g; g += 2) {
            group(vrA, r_lo + 16 * g);
            if (g + 2 < n_g) load_v(vrA, r_lo + 16 * (g + 2));
            if (g + 1 < n_g) {
                group(vrB, r_lo + 16 * (g + 1));
                if (g + 3 < n_g) load_v(vrB, r_lo + 16 * (g + 3));
            }
        }
    }
    // C layout: lane (n, kg) holds dims 16 i + 4 kg .. + 3 of head n
    if (half == 1 && n < 6) {
#pragma unroll
        for (int i = 0; i < 16; i++)
            *reinterpret_cast<f4*>(&sacc[(hk * 6 + n) * 256 + 16 * i + 4 * kg]) = o[i];
    }
    __syncthreads();
    if (half == 0 && n < 6) {
        const int hq = hk * 6 + n;
        float* out = a.part + ((size_t)hq * a.part_stride + part_idx) * 258;
        typedef float f2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const f4 h1 = *reinterpret_cast<const f4*>(&sacc[(hk * 6 + n) * 256 + 16 * i + 4 * kg]);
            const int d = 16 * i + 4 * kg;
            stg<f2>(&out[d], f2{o[i][0] + h1[0], o[i][1] + h1[1]});
            stg<f2>(&out[d + 2], f2{o[i][2] + h1[2], o[i][3] + h1[3]});
        }
        if (kg == 0) {
            stg<float>(&out[256], sml[hq * 2 + 0]);
            stg<float>(&out[257], sml[hq * 2 + 1]);
        }
    }
}

// One block of work: compressed chunk `chunk` of the sequence described by a
// (chunk == n_chunks: its raw window).
__device__ __forceinline__ void ws_block(const AttnArgs& a, int chunk, int tiles_per_chunk,
                                         int n_chunks) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    Smem& S = *reinterpret_cast<Smem*>(smem_raw);
    const int tid = threadIdx.x;
    const int wv = tid >> 6;
    const int h = wv & 3;
    const int lane = tid & 63;
    if (chunk >= n_chunks) {  // the window block(s) after the compressed chunks
#ifdef KHQ_PHASE_TIMING
        const unsigned long long wt0 = __builtin_amdgcn_s_memrealtime();
#endif
        if (a.win_blocks == NWIN)
            window_block(a, S, a.part_offset + n_chunks, chunk - n_chunks);
        else
            window_block_all(a, S, a.part_offset + n_chunks);
#ifdef KHQ_PHASE_TIMING
        if (threadIdx.x == 0 && blockIdx.x < 1024) {
            block_times[blockIdx.x][0] = wt0;
            block_times[blockIdx.x][1] = __builtin_amdgcn_s_memrealtime();
        }
#endif
        return;
    }
    const int c_len = a.c_len;
    int s_lo, s_hi;
    if (a.split_per > 0) {  // the reference's split partition, cut into chunks
        const int sp = chunk / a.split_subs, sub = chunk - sp * a.split_subs;
        const int lo = min(sp * a.split_per, c_len), hi = min(lo + a.split_per, c_len);
        s_lo = min(lo + sub * tiles_per_chunk * TT, hi);
        s_hi = min(s_lo + tiles_per_chunk * TT, hi);
    } else {
        s_lo = min(chunk * tiles_per_chunk * TT, c_len);
        s_hi = min(s_lo + tiles_per_chunk * TT, c_len);
    }
    const int n_tiles = (s_hi - s_lo + TT - 1) / TT;
#ifdef KHQ_PHASE_TIMING
    unsigned long long ph_t = __builtin_amdgcn_s_memtime();
    const unsigned long long rt0 = __builtin_amdgcn_s_memrealtime();
    unsigned ph_acc[32];
#pragma unroll
    for (int k = 0; k < 32; k++) ph_acc[k] = 0;
#endif

    // ---- shared tables: the sign and outlier selector tables are computed
    // here; cents_k[2], the rotors, d_v, cents_v[.][4 p + 3] and the RoPE
    // table are loaded here and stored after the query transforms (the
    // value wavefronts copy the codebook after the first block barrier)
    SetupIn in;
    TabIn tb;
    {
        load_setup(a, h, wv, lane, in);
        load_tables(a, tid, tb);
        PHASE(24);
        // key wavefronts: sign tables; value wavefronts: outlier selectors
        // (a wavefront-uniform split)
        const int t = tid & 255;
        if (tid < 4) {
            S.kdone[tid] = 0;
            S.vread[tid] = 0;
        }
        if (tid == 0) S.fault = 0;
        if (wv < 4) {
            // mask byte t (codes of 4 dims): sign halves (code 1 -> -1, codes
            // 2 and 3 -> +1; an outlier's own sign is OR-ed in from its window
            // half) and, per output word (dims 0, 1 | dims 2, 3), the byte
            // selectors of the window halves: the d-th outlier of the byte
            // takes window half d (bytes 2 d, 2 d + 1), other dims 0x0C (zero).
            uint32_t sg[2], sl[2];
            int r = 0;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                uint32_t g = 0u, n = 0x0C0C0C0Cu;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int code = (t >> (2 * (2 * k + e))) & 3;
                    const uint32_t hv = code == 1 ? 0xBC00u : (code >= 2 ? 0x3C00u : 0u);
                    g |= hv << (16 * e);
                    if (code == 3) {
                        n = (n & ~(0xFFFFu << (16 * e))) |
                            (((uint32_t)(2 * r) | ((uint32_t)(2 * r + 1) << 8)) << (16 * e));
                        r++;
                    }
                }
                sg[k] = g;
                sl[k] = n;
            }
            S.ktab[t] = uint4{sg[0], sg[1], sl[0], sl[1]};
            uint32_t f0 = 0u, f1 = 0u;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                f0 |= ((t >> k) & 1) ? 0x80u << (8 * k) : 0u;
                f1 |= ((t >> (4 + k)) & 1) ? 0x80u << (8 * k) : 0u;
            }
            S.sgb[t] = uint2{f0, f1};
        } else {
            // the constant tail of every rank-window row (ranks 56 ..) and the
            // two zero words of every staged kpay row
#pragma unroll
            for (int i = 0; i < 3; i++) {
                const int x = t + 256 * i;  // 768 = 4 heads x 16 tokens x 12 ranks
                const int row = x / 12, r = 56 + x % 12;
                (&S.ke[0][0])[row * KE_S + r] = 0x80008000u;
            }
            if (t < 128) (&S.kp[0][0])[(t >> 1) * KP_TS + 10 + (t & 1)] = 0u;
        }
    }

    PHASE(0);

    if (wv < 4) {
        key_role(a, S, in, tb, h, lane, s_lo, s_hi, n_tiles PH_ARGS);
    } else {
        value_role(a, S, in, tb, h, lane, s_lo, s_hi, n_tiles PH_ARGS);
    }
#ifdef KHQ_PHASE_TIMING
    ph_t = __builtin_amdgcn_s_memtime();
#endif

    // ---- output: wavefront wv handles query heads 3 (wv / 4) .. + 2 of KV head h
    // (S.fault is final: every wait precedes the roles' last block barrier)
    const bool bad = __hip_atomic_load(&S.fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
    if (bad && tid == 0) atomicOr(&g_fault, 1);
    const float* ep = S.o[h];
    float rv[16];
#pragma unroll
    for (int t = 0; t < 16; t++) rv[t] = (float)S.rotv[lane * 16 + t];
    float rdv[4];
#pragma unroll
    for (int c = 0; c < 4; c++)  // hardware reciprocal: 1 ulp, far below the output bar
        rdv[c] = 0.0625f * __builtin_amdgcn_rcpf((float)S.dvh[lane * 4 + c] + 1e-8f);
    PHASE(25);
#pragma unroll
    for (int hh = 0; hh < 3; hh++) {
        const int hd = 3 * (wv >> 2) + hh;
        float o[4], u[4];
#pragma unroll
        for (int c = 0; c < 4; c++) o[c] = ep[hd * 256 + lane * 4 + c];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float t = o[0] * rv[c * 4 + 0];
            t = fmaf(o[1], rv[c * 4 + 1], t);
            t = fmaf(o[2], rv[c * 4 + 2], t);
            t = fmaf(o[3], rv[c * 4 + 3], t);
            u[c] = t;
        }
        fwht256(u, lane);
        PHASE(26);
        const int hq = h * 6 + hd;
        float* out = a.part + ((size_t)hq * a.part_stride + a.part_offset + chunk) * 258;
        const float M = bad ? __builtin_nanf("") : S.ml[h][hd][0];
        const float L = S.ml[h][hd][1];
        const bool empty = (M == -INFINITY);
        // partial rows are 258 floats: 8-byte aligned, so 8-byte stores
        typedef float f2 __attribute__((ext_vector_type(2)));
        stg<f2>(&out[lane * 4], empty ? f2{0.f, 0.f} : f2{u[0] * rdv[0], u[1] * rdv[1]});
        stg<f2>(&out[lane * 4 + 2], empty ? f2{0.f, 0.f} : f2{u[2] * rdv[2], u[3] * rdv[3]});
        if (lane == 0) stg<f2>(&out[256], empty ? f2{-1e20f, 0.f} : f2{M, L});
    }
    PHASE(15);
#ifdef KHQ_PHASE_TIMING
    if ((threadIdx.x & 0xFF) == 0)
        for (int k = 0; k < 32; k++) atomicAdd(&phase_cycles[k], (unsigned long long)ph_acc[k]);
    if (threadIdx.x == 0 && blockIdx.x < 1024) {
        block_times[blockIdx.x][0] = rt0;
        block_times[blockIdx.x][1] = __builtin_amdgcn_s_memrealtime();
    }
#endif
}

__global__ __launch_bounds__(NTHR, 1) void attn_ws_kernel(AttnArgs a, int tiles_per_chunk,
                                                          int n_chunks) {
    ws_block(a, blockIdx.x, tiles_per_chunk, n_chunks);
}

// Batched form: block b works on sequence map[b].x, chunk map[b].y (the
// sequence's n_parts compressed chunks, then its window block).
__global__ __launch_bounds__(NTHR, 1) void attn_ws_batched_kernel(const AttnArgs* __restrict__ args,
                                                                  const int2* __restrict__ map) {
    const int2 m = map[blockIdx.x];
    const AttnArgs& a = args[m.x];  // read in place (a private copy would go to scratch)
    ws_block(a, m.y, a.chunk_tiles, a.n_parts);
}

}  // namespace ws

static_assert((4 * 6 * 256 + 4 * 6 * 2 + 4 * 6 * 256) * sizeof(float) + 8 * 256 * 20 * 2 <=
                  sizeof(ws::Smem),
              "window block LDS: scores, sums, half-sums and V^T staging fit the block's LDS");
size_t attn_ws_smem_bytes() { return sizeof(ws::Smem); }

std::atomic<int> g_spin_limit{1 << 20};

// Chunking of the compressed region: at most n_cu - 1 chunks (one CU left for
// the window), each of the same whole number of tiles.  When that leaves no
// room for the NWIN per-KV-head window blocks and the chunks are short (a
// chunk of p tiles takes about 10 + 2.3 p us, the single all-heads window
// block about 23 us), the cap drops to n_cu - NWIN so the four window blocks
// run beside the chunks instead.
int attn_ws_tiles_per_chunk(int c_len, int* n_chunks) {
    static const int env_max = [] {
        const char* e = getenv("KHQ_MAX_CHUNKS");
        return e ? atoi(e) : 0;
    }();
    const int n_cu = device_cu_count();
    const int tiles = (c_len + ws::TT - 1) / ws::TT;
    auto split = [tiles](int max_chunks, int* n) {
        int chunks = tiles < max_chunks ? tiles : max_chunks;
        if (chunks < 1) chunks = 1;
        const int per = (tiles + chunks - 1) / chunks;
        *n = (tiles + per - 1) / per;
        return per;
    };
    if (env_max > 0) return split(env_max, n_chunks);
    int per = split(n_cu > 1 ? n_cu - 1 : 1, n_chunks);
    if (*n_chunks + ws::NWIN > n_cu && per <= 4 && n_cu > ws::NWIN) per = split(n_cu - ws::NWIN, n_chunks);
    return per;
}

void fill_rope_table(AttnArgs& a) {
    // freq = powf(base, -2 m / 64) as the oracle and the portable kernels
    // compute it; the 16-token rotation in double, rounded once
    thread_local float last_base = -1.0f;
    thread_local float tab[96];
    if (a.rope_base != last_base) {
        for (int g = 0; g < 4; g++)
            for (int u = 0; u < 8; u++) {
                const int m = 16 * (u >> 2) + 4 * g + (u & 3);
                const float f = powf(a.rope_base, -2.0f * (float)m / 64.0f);
                tab[(g * 3 + 0) * 8 + u] = f;
                tab[(g * 3 + 1) * 8 + u] = (float)cos(16.0 * (double)f);
                tab[(g * 3 + 2) * 8 + u] = (float)sin(16.0 * (double)f);
            }
        last_base = a.rope_base;
    }
    memcpy(a.rope_tab, tab, sizeof(tab));
}

hipError_t launch_attn_ws(const AttnArgs& a, int tiles_per_chunk, int n_chunks, hipStream_t st) {
    const size_t smem = sizeof(ws::Smem);
    hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&ws::attn_ws_kernel), (int)smem);
    if (e != hipSuccess) return e;
    // four window blocks when they fit beside the chunks, else one (it is
    // hidden behind chunks of several tiles then)
    const int n_cu = device_cu_count();
    AttnArgs b = a;
    b.win_blocks = n_chunks + ws::NWIN <= n_cu ? ws::NWIN : 1;
    const int blocks = n_chunks + (a.win_len > 0 ? b.win_blocks : 0);
    fill_rope_table(b);
    b.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
    hipLaunchKernelGGL(ws::attn_ws_kernel, dim3(blocks), dim3(ws::NTHR), smem, st, b,
                       tiles_per_chunk, n_chunks);
    return hipGetLastError();
}

hipError_t launch_attn_ws_batched(const AttnArgs* args, const int2* map, int n_blocks,
                                  hipStream_t st) {
    const size_t smem = sizeof(ws::Smem);
    hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&ws::attn_ws_batched_kernel),
                                      (int)smem);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(ws::attn_ws_batched_kernel, dim3(n_blocks), dim3(ws::NTHR), smem, st,
                       args, map);
    return hipGetLastError();
}

hipError_t fault_status(int* out, int clear) {
    hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(ws::g_fault), sizeof(int));
    if (e == hipSuccess && clear && *out) {
        const int z = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(ws::g_fault), &z, sizeof(int));
    }
    return e;
}

}  // namespace khq

#ifdef KHQ_PHASE_TIMING
extern "C" int khq_ws_phase_cycles(unsigned long long* out, int reset) {
    hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(khq::ws::phase_cycles),
                                       sizeof(unsigned long long) * 32);
    if (e == hipSuccess && reset) {
        unsigned long long z[32] = {0};
        e = hipMemcpyToSymbol(HIP_SYMBOL(khq::ws::phase_cycles), z, sizeof(z));
    }
    return e == hipSuccess ? 0 : (int)e;
}
extern "C" int khq_ws_block_times(unsigned long long* out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(khq::ws::block_times),
                                    sizeof(unsigned long long) * 2048);
}
#endif
