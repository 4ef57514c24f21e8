// khq_prefill.hip -- chunked prefill on matrix cores: many query tokens of one
// layer attend to the compressed prefix and the raw ring window at once.
//
// Kernels that build one dense fp16 key space (key index = token position)
// and attend over it causally:
//   decompress_kernel   compressed rows -> roped K rows [key][H_kv][256] and
//                       V^T [H_kv][256][ld] (the decode of the compressed-
//                       region attention kernel, ref:src/csrc/
//                       qmv_sm75_kernel.cu:1608-1699 for K and :1739-1762,
//                       1776-1826 for V, applied per token instead of being
//                       folded into the running sums);
//   ring_gather_kernel  raw ring slots -> the same K rows / V^T columns;
//   compress_decode_kernel  a compression event that decodes the rows it
//                       packs into the key space (and appends new tokens);
//   prefill_attn_kernel, prefill_attn_rs_kernel  S^T = K Q^T and
//                       O^T = V^T P^T on MFMA (fp16 in, fp32 accumulate),
//                       online softmax, one split of the keys per block;
//   prefill_merge_kernel  the splits' partial triples merged and gated.
// Query j of a launch sees keys [0, vis0 + j): the sequential step semantics
// (its own position included) when keys are positions.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <algorithm>

#include "khq_internal.h"
#include "khq_mfma_util.h"
#include "khq_decode_row.h"
#include "khq_compress_row.h"

namespace khq {
namespace pf {

using namespace mu;

constexpr int TOK_BLK = 4;    // tokens per decompress / gather block: one per wavefront
                              // (small blocks spread a short chunk over many CUs)
constexpr int BLK_THR = 64 * TOK_BLK;
constexpr int VT_PAD = 8;     // halves of padding per LDS V^T row

__device__ __forceinline__ uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Writes the block's LDS V^T tile sv[256][TOK_BLK + VT_PAD] to vt columns
// key0 .. key0 + TOK_BLK - 1 of KV head h (all TOK_BLK columns: the caller's
// buffer is padded to a multiple of 64 keys), in 8-byte pieces (key0 is a
// multiple of 4).
__device__ __forceinline__ void store_vt(const _Float16 (*sv)[TOK_BLK + VT_PAD], __half* vt, int ld,
                                         int h, int key0) {
    for (int i = threadIdx.x; i < 256 * (TOK_BLK / 4); i += blockDim.x) {
        const int d = i / (TOK_BLK / 4), part = i % (TOK_BLK / 4);
        const uint2 v = *reinterpret_cast<const uint2*>(&sv[d][part * 4]);
        *reinterpret_cast<uint2*>(vt + ((size_t)h * 256 + d) * ld + key0 + part * 4) = v;
    }
}

// Writes columns key0 .. key0 + nc - 1 only (any alignment), 2 bytes each.
__device__ __forceinline__ void store_vt_cols(const _Float16 (*sv)[TOK_BLK + VT_PAD], __half* vt,
                                              int ld, int h, int key0, int nc) {
    for (int i = threadIdx.x; i < 256 * TOK_BLK; i += blockDim.x) {
        const int d = i / TOK_BLK, c = i % TOK_BLK;
        if (c < nc)
            reinterpret_cast<_Float16*>(vt)[((size_t)h * 256 + d) * ld + key0 + c] = sv[d][c];
    }
}

// ------------------------------------------------------------- decompress
// Block (16 tokens, KV head h), one wavefront per token (the decode of one
// row is a chain of dependent loads: tokens in parallel hide it); lane p owns
// patch p = dims 4 p .. 4 p + 3.
__device__ __forceinline__ void decompress_block(const DecompArgs& a, int bx, int h) {
    __shared__ __align__(16) _Float16 sv[256][TOK_BLK + VT_PAD];
    const int wv = threadIdx.x >> 6, p = threadIdx.x & 63;
    const int t_blk = bx * TOK_BLK;
    dec::Consts cs;
    dec::load_consts(a, p, cs);
    {
        const int tl = wv;           // token within the block
        const int tok = t_blk + tl;
        if (tok >= a.n_tok) {        // uniform per wavefront
#pragma unroll
            for (int c = 0; c < 4; c++) sv[4 * p + c][tl] = (_Float16)0.0f;
            goto staged;
        }
        const size_t g = (size_t)(a.tok0 + tok) * a.h_kv + h;
        float y[4];
        // ---- K: codes, outlier ordinals (ballot prefix), values, RoPE
        dec::decode_k(a, cs, a.kmask[g * 16 + (p >> 2)], a.kpay + g * 40, __half2float(a.knorm[g]),
                      __half2float(a.krn[g]), (float)(a.start_pos + a.tok0 + tok), p, y);
        *reinterpret_cast<uint2*>(a.out_k + ((size_t)(a.key0 + tok) * a.h_kv + h) * 256 + 4 * p) =
            uint2{pk_rne(y[0], y[1]), pk_rne(y[2], y[3])};
        // ---- V: patch fields, codebook, dim 3, inverse rotor, FWHT
        const uint8_t* vp = a.vpay + g * 104;
        const uint32_t grp = (uint32_t)p / 8, sub = (uint32_t)p % 8;
        const uint64_t w0 = rd32(vp + (grp * 3 + 0) * 4), w1 = rd32(vp + (grp * 3 + 1) * 4),
                       w2 = rd32(vp + (grp * 3 + 2) * 4);
        const uint64_t low64 = (w1 << 32) | w0, high64 = (w2 << 32) | w1;
        const uint32_t pvl = (sub < 4) ? (uint32_t)((low64 >> (sub * 12)) & 0xFFF)
                                       : (uint32_t)((high64 >> ((sub - 4) * 12 + 16)) & 0xFFF);
        const uint32_t hb = (p < 32) ? ((rd32(vp + 96) >> p) & 1u) : ((rd32(vp + 100) >> (p - 32)) & 1u);
        dec::decode_v(a, cs, (pvl & 0x7Fu) | (hb << 7), pvl, __half2float(a.vnorm[g]),
                      __half2float(a.vrn[g]), __uint_as_float(rd32(a.vsm + g * 4)), p, y);
#pragma unroll
        for (int c = 0; c < 4; c++) sv[4 * p + c][tl] = (_Float16)y[c];
    }
staged:
    __syncthreads();
    store_vt(sv, a.out_vt, a.ld_vt, h, a.key0 + t_blk);
}

// ------------------------------------------------------------ ring gather
// Block (16 keys, KV head h), one wavefront per key: K rows copied, V rows
// transposed through LDS.  In chunk mode the keys come from the caller's new
// tokens, which also go to their ring slots (one launch appends a chunk to
// the ring and to the dense key space).
__device__ __forceinline__ void gather_block(const GatherArgs& a, int bx, int h, int bz) {
    __shared__ __align__(16) _Float16 sv[256][TOK_BLK + VT_PAD];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t_blk = bx * TOK_BLK;
    // job 0: the gather / chunk write; job 1: the side copy (block-uniform)
    const bool side = bz == 1;
    const int n = side ? a.side_n : a.n;
    const int key0 = side ? a.side_key0 : a.key0;
    if (t_blk >= n) return;
    {
        const int tl = wv;
        const int t = t_blk + tl;
        if (t >= n) {
#pragma unroll
            for (int c = 0; c < 4; c++) sv[4 * lane + c][tl] = (_Float16)0.0f;
            goto staged;
        }
        uint2 kw, vw;
        if (side) {
            if (t >= a.side_from_src) {
                const size_t cs = ((size_t)(t - a.side_from_src) * a.h_kv + h) * 256 + 4 * lane;
                kw = *reinterpret_cast<const uint2*>(a.src_k + cs);
                vw = *reinterpret_cast<const uint2*>(a.src_v + cs);
            } else {
                int slot = a.side_start + t;
                slot = slot >= a.ring_cap ? slot - a.ring_cap : slot;
                const size_t rs = ((size_t)slot * a.h_kv + h) * 256 + 4 * lane;
                kw = *reinterpret_cast<const uint2*>(a.wr_k + rs);
                vw = *reinterpret_cast<const uint2*>(a.wr_v + rs);
            }
        } else {
            int slot = a.win_start + t;
            slot = slot >= a.ring_cap ? slot - a.ring_cap : slot;
            const size_t rs = ((size_t)slot * a.h_kv + h) * 256 + 4 * lane;
            if (a.src_k) {
                const size_t cs = ((size_t)t * a.h_kv + h) * 256 + 4 * lane;
                kw = *reinterpret_cast<const uint2*>(a.src_k + cs);
                vw = *reinterpret_cast<const uint2*>(a.src_v + cs);
                *reinterpret_cast<uint2*>(a.wr_k + rs) = kw;
                *reinterpret_cast<uint2*>(a.wr_v + rs) = vw;
                if (a.wr_u) *reinterpret_cast<uint2*>(a.wr_u + rs) = *reinterpret_cast<const uint2*>(a.src_u + cs);
            } else {
                kw = *reinterpret_cast<const uint2*>(a.ring_k + rs);
                vw = *reinterpret_cast<const uint2*>(a.ring_v + rs);
            }
        }
        *reinterpret_cast<uint2*>(a.out_k + ((size_t)(key0 + t) * a.h_kv + h) * 256 + 4 * lane) = kw;
        const h4 v = __builtin_bit_cast(h4, vw);
#pragma unroll
        for (int c = 0; c < 4; c++) sv[4 * lane + c][tl] = v[c];
    }
staged:
    __syncthreads();
    if (a.src_k)  // chunk mode: exactly the written columns (key0 is any position)
        store_vt_cols(sv, a.out_vt, a.ld_vt, h, key0 + t_blk, min(TOK_BLK, n - t_blk));
    else
        store_vt(sv, a.out_vt, a.ld_vt, h, key0 + t_blk);
}

__global__ __launch_bounds__(BLK_THR) void decompress_kernel(DecompArgs a) {
    decompress_block(a, blockIdx.x, blockIdx.y);
}

__global__ __launch_bounds__(BLK_THR) void ring_gather_kernel(GatherArgs a) {
    gather_block(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

// A decode and an independent gather (disjoint outputs, no data passed
// between them) in one launch: blocks [0, nb_d) decode (x fastest, then the
// KV head), the rest gather (x, then the KV head, then the job plane).
__global__ __launch_bounds__(BLK_THR) void decompress_gather_kernel(DecompArgs d, GatherArgs g,
                                                                    int nx_d, int nx_g) {
    const int nb_d = nx_d * d.h_kv;
    int b = blockIdx.x;
    if (b < nb_d) {
        decompress_block(d, b % nx_d, b / nx_d);
        return;
    }
    b -= nb_d;
    const int per_plane = nx_g * g.h_kv;
    const int bz = b / per_plane;
    b -= bz * per_plane;
    gather_block(g, b % nx_g, b / nx_g, bz);
}

// A compression event, the decode of its rows into the dense key space and
// an independent gather (a chunk append or a raw copy, disjoint from the
// rows compressed) in one launch: blocks [0, nb_k) compress and decode K rows
// (four per block, the longest blocks, first), [nb_k, nb_k + n_v) V rows (one
// per block), the rest gather (x, then the KV head, then the job plane;
// nx_g = 0: no gather).
__global__ __launch_bounds__(BLK_THR) void compress_decode_kernel(CompressJob k, CompressJob v,
                                                                  DecompArgs d, GatherArgs g,
                                                                  int nb_k, int nx_g) {
    int b = blockIdx.x;
    if (b < nb_k) {
        compress_block<true>(k.x, k.d_vec, k.rotor, k.cents, k.vq, k.out_mask, k.out_norms,
                             k.out_rn, k.out_pay, nullptr, k.n, k.ts, k.alpha, 0, b, &d);
        return;
    }
    b -= nb_k;
    if (b < v.n) {
        compress_block<true>(v.x, v.d_vec, v.rotor, v.cents, v.vq, v.out_mask, v.out_norms,
                             v.out_rn, v.out_pay, v.out_sm, v.n, v.ts, v.alpha, 1, b, &d);
        return;
    }
    b -= v.n;
    const int per_plane = nx_g * g.h_kv;
    const int bz = b / per_plane;
    b -= bz * per_plane;
    gather_block(g, b % nx_g, b / nx_g, bz);
}

// Visibility of the keys of one 32-key tile to one query row, as a bit mask
// (bit i: key k0 + i): [0, vis) less the hole, plus the extra range (hole and
// extra are empty for rows after a compression event).  Only vis and a lane
// flag stay live; the hole and extra bounds are the launch's scalar arguments.
__device__ __forceinline__ uint32_t bits_below(int n) {  // bits [0, n) of 32
    return n >= 32 ? ~0u : (n <= 0 ? 0u : (1u << n) - 1u);
}
struct RowKeys {
    const PrefillArgs& a;
    int vis;
    bool run_a;
    __device__ __forceinline__ RowKeys(const PrefillArgs& a_, bool r_ok, int jq) : a(a_) {
        // padding rows see every key: their scores are never written
        vis = r_ok ? min(a.n_k, a.vis0 + jq) : a.n_tot;
        run_a = r_ok && jq < a.q_b;
    }
    __device__ __forceinline__ uint32_t tile(int k0) const {
        // selects, no branch: a divergent branch here costs the 32-row
        // kernel about 45 registers (spilled to AGPRs)
        const uint32_t hole = bits_below(a.hole_hi - k0) & ~bits_below(a.hole_lo - k0);
        // extra key ex_lo + i stands for position hole_lo + i: visible below vis
        const int ex_end = min(a.ex_hi, a.ex_lo + vis - a.hole_lo);
        const uint32_t ex = bits_below(ex_end - k0) & ~bits_below(a.ex_lo - k0);
        const uint32_t m = bits_below(vis - k0);
        return run_a ? ((m & ~hole) | ex) : m;
    }
};
// One past the last key any row of the block sees (rows are ordered by query).
__device__ __forceinline__ int block_key_end(const PrefillArgs& a, int row_first, int row_last) {
    int lim = min(a.n_k, a.vis0 + row_last / a.n_rep);
    if (row_first / a.n_rep < a.q_b) lim = max(lim, a.ex_hi);
    return lim;
}

// ----------------------------------------------------------- attention
// Block = 4 wavefronts = 4 tiles of 16 query rows of one KV head, one key
// split.  Row r of KV head h is (query j = r / n_rep, head h n_rep + r % n_rep).
// Per 32-key tile the block stages K (32 x 256) and V^T (256 x 32) in LDS
// (double-buffered, one barrier per tile; the next tile's global loads are in
// flight while this one is computed), then each wavefront computes
//   S^T (two 16-key halves x 16 rows) = 16 MFMA 16x16x32, A = K rows, B = Q^T
//   (registers); lane (row li, lg) gets keys 4 lg .. 4 lg + 3 of each half;
//   O^T (256 dims x 16 rows) += 16 MFMA 16x16x32 with K = the tile's 32 keys
//   in the order (4 lg .. 4 lg + 3, 16 + 4 lg .. 16 + 4 lg + 3) per lane
//   group, so P^T is the S^T C layout as is and A = V^T read in that order.
// Softmax: a per-row reference maximum shared by the row's 4 lanes, raised
// (with a cross-lane reduction and a rescale) only when a score exceeds it by
// more than 8, so weights stay <= e^8; row sums are per lane until the end.
constexpr int KT = 32;            // keys per tile
constexpr int KS_LD = 256 + 16;   // halves per LDS K row (bank spread measured with
                                  // SQ_LDS_BANK_CONFLICT)
constexpr int VS_LD = KT + 4;     // halves per LDS V^T row (rows 8-byte aligned:
                                  // stored and read in 8-byte pieces)
constexpr float GAP = 8.0f;

__global__ __launch_bounds__(256) void prefill_attn_kernel(PrefillArgs a) {
    __shared__ __align__(16) _Float16 ks[2][KT][KS_LD];
    __shared__ __align__(16) _Float16 vs[2][256][VS_LD];
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int wv = tid >> 6, lane = tid & 63;
    const int li = lane & 15, lg = lane >> 4;
    const int n_rows = a.n_q * a.n_rep;
    const int row0 = (blockIdx.x * 4 + wv) * 16;
    const int split = blockIdx.z;
    const int k_lo = split * a.keys_per_split;
    const int k_hi = min(a.n_tot, k_lo + a.keys_per_split);
    const int H_q = a.h_kv * a.n_rep;
    const int r = row0 + li;
    const bool r_ok = r < n_rows;
    const int jq = r_ok ? r / a.n_rep : 0;
    const int hq = h * a.n_rep + (r_ok ? r % a.n_rep : 0);
    const RowKeys vis(a, r_ok, jq);
    const int b_last = min((int)blockIdx.x * 64 + 63, n_rows - 1);
    const int kt_hi = min(k_hi, block_key_end(a, blockIdx.x * 64, b_last));

    h8 qb[8];
    {
        const __half* qrow = a.q + ((size_t)jq * H_q + hq) * 512;
#pragma unroll
        for (int st = 0; st < 8; st++) {
            const uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * st + 8 * lg);
            qb[st] = __builtin_bit_cast(h8, r_ok ? v : uint4{0u, 0u, 0u, 0u});
        }
    }
    f4 acc[16];
#pragma unroll
    for (int m = 0; m < 16; m++) acc[m] = f4{0.f, 0.f, 0.f, 0.f};
    float m_ref = -INFINITY, l_part = 0.0f;

    // cooperative tile loads: thread t -> K key t / 8, 64 B at (t % 8) * 32
    // halves; V^T dim t, the tile's 32 keys (64 B)
    const int ld_key = tid >> 3, ld_off = (tid & 7) * 32;
    const __half* kg = a.k + (size_t)h * 256 + ld_off;
    const __half* vg = a.vt + ((size_t)h * 256 + tid) * a.ld_vt;
    uint4 pk[4], pv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pk[i] = pv[i] = uint4{0u, 0u, 0u, 0u};
    auto gload = [&](int k0) {
        const int key = min(k0 + ld_key, a.n_tot - 1);
        const uint4* ksrc = reinterpret_cast<const uint4*>(kg + (size_t)key * a.h_kv * 256);
        const uint4* vsrc = reinterpret_cast<const uint4*>(vg + k0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pk[i] = ksrc[i];
            pv[i] = vsrc[i];
        }
    };
    // V^T word w of a tile row holds keys 2 w, 2 w + 1; columns past n_k are
    // padding and become zero
    auto vmask = [](uint32_t w, int i, int nv) {
        return 2 * i + 1 < nv ? w : (2 * i < nv ? (w & 0xFFFFu) : 0u);
    };
    auto lstore = [&](int buf, int k0) {
        const int nv = a.n_tot - k0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *reinterpret_cast<uint4*>(&ks[buf][ld_key][ld_off + 8 * i]) = pk[i];
            uint4 v = pv[i];
            if (nv < KT)
                v = uint4{vmask(v.x, 4 * i, nv), vmask(v.y, 4 * i + 1, nv), vmask(v.z, 4 * i + 2, nv),
                          vmask(v.w, 4 * i + 3, nv)};
            *reinterpret_cast<uint2*>(&vs[buf][tid][8 * i]) = uint2{v.x, v.y};
            *reinterpret_cast<uint2*>(&vs[buf][tid][8 * i + 4]) = uint2{v.z, v.w};
        }
    };

    const int n_tiles = k_lo < kt_hi ? (kt_hi - k_lo + KT - 1) / KT : 0;
    if (n_tiles > 0) {
        gload(k_lo);
        lstore(0, k_lo);
        if (n_tiles > 1) gload(k_lo + KT);
    }
    __syncthreads();
    for (int t = 0; t < n_tiles; t++) {
        const int buf = t & 1;
        const int k0 = k_lo + t * KT;
        // ---- S^T of both 16-key halves from LDS
        f4 s0 = f4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int st = 0; st < 8; st++) {
            const h8 ka = *reinterpret_cast<const h8*>(&ks[buf][li][32 * st + 8 * lg]);
            const h8 kb = *reinterpret_cast<const h8*>(&ks[buf][16 + li][32 * st + 8 * lg]);
            s0 = mfma32(ka, qb[st], s0);
            s1 = mfma32(kb, qb[st], s1);
        }
        float sc[8], lmax = -INFINITY;
        {
            const uint32_t mb = vis.tile(k0) >> (4 * lg);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                sc[c] = (mb >> c) & 1u ? s0[c] * a.sc : -INFINITY;
                sc[4 + c] = (mb >> (16 + c)) & 1u ? s1[c] * a.sc : -INFINITY;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) lmax = fmaxf(lmax, sc[e]);
        // ---- raise the row's reference maximum only when needed
        if (__ballot(lmax > m_ref + GAP) != 0ull) {
            float rmax = fmaxf(lmax, __shfl_xor(lmax, 16, 64));
            rmax = fmaxf(rmax, __shfl_xor(rmax, 32, 64));
            const float m_new = fmaxf(m_ref, rmax);
            if (m_new > m_ref) {
                const float fac = __expf(m_ref - m_new);  // 0 when m_ref = -inf
#pragma unroll
                for (int m = 0; m < 16; m++) acc[m] *= fac;
                l_part *= fac;
                m_ref = m_new;
            }
        }
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            p[e] = sc[e] == -INFINITY ? 0.0f : __expf(sc[e] - m_ref);
            l_part += p[e];
        }
        const h8 pb = __builtin_bit_cast(
            h8, uint4{pk_rne(p[0], p[1]), pk_rne(p[2], p[3]), pk_rne(p[4], p[5]), pk_rne(p[6], p[7])});
        // ---- O^T += V^T P^T (K = the 32 keys in the lane order above)
#pragma unroll
        for (int m4 = 0; m4 < 16; m4 += 4) {  // 4 operand reads in flight, then 4 MFMAs
            h8 vop[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint2 va = *reinterpret_cast<const uint2*>(&vs[buf][16 * (m4 + i) + li][4 * lg]);
                const uint2 vb = *reinterpret_cast<const uint2*>(&vs[buf][16 * (m4 + i) + li][16 + 4 * lg]);
                vop[i] = __builtin_bit_cast(h8, uint4{va.x, va.y, vb.x, vb.y});
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the 4 reads ahead of their MFMAs
#pragma unroll
            for (int i = 0; i < 4; i++) acc[m4 + i] = mfma32(vop[i], pb, acc[m4 + i]);
        }
        // ---- stage the next tile, load the one after
        if (t + 1 < n_tiles) {
            lstore(buf ^ 1, k0 + KT);
            if (t + 2 < n_tiles) gload(k0 + 2 * KT);
        }
        __syncthreads();
    }
    // ---- partial triple of row li (dims 16 mt + 4 lg + c)
    float l_row = l_part + __shfl_xor(l_part, 16, 64);
    l_row += __shfl_xor(l_row, 32, 64);
    if (r_ok) {
        float* out = a.part + ((size_t)(jq * H_q + hq) * a.n_split + split) * 258;
        const bool empty = (m_ref == -INFINITY);
#pragma unroll
        for (int mt = 0; mt < 16; mt++)
            *reinterpret_cast<f4*>(&out[16 * mt + 4 * lg]) = empty ? f4{0.f, 0.f, 0.f, 0.f} : acc[mt];
        if (lg == 0) {
            out[256] = empty ? -1e20f : m_ref;
            out[257] = empty ? 0.0f : l_row;
        }
    }
}

// 32-row form: 32 query rows per wavefront pair on 32x32x16 MFMAs, so every
// K / V^T operand read from LDS feeds twice the arithmetic of the 16-row
// form; the O^T accumulators (32 rows x 256 dims) and Q^T (32 x 256 fp16)
// stay in registers, split between the pair.  32x32 layouts (lane l,
// n = l % 32, hh = l / 32):
//   A[m][k]: lane m + 32 (k / 8) holds element k % 8;  B[k][n] likewise;
//   C[m][n]: lane n + 32 hh, register r <-> m = 8 (r / 4) + 4 hh + r % 4.
// S^T = K Q^T (keys x rows); its C registers 8 s' .. 8 s' + 7 are the B
// operand of K-step s' of O^T += V^T P^T when that step's K order is
// key 8 (2 s' + i / 4) + 4 hh + i % 4 for element i, which is how V^T is read.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16 mfma3232(h8 a, h8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
constexpr int KS2_LD = 256 + 8;   // halves per LDS K row
constexpr int VS2_LD = KT + 4;    // halves per LDS V^T row

constexpr int NKB = 3;            // LDS tile slots
// Lazy-rescale gap of the 32-row form: weights stay <= e^10 (< fp16 max).
constexpr float GAP32 = 10.0f;

// Role-specialised 32-row attention: per SIMD a score wavefront and an
// output wavefront (8 wavefronts per block, 128 rows of one KV head).  The
// score wavefront of row group g computes S^T = K Q^T (tile t + 1 on the
// matrix cores while tile t is masked, scaled and its row maximum taken),
// decides whether the row's reference maximum rises (rescale factor fac) and
// leaves tile t's masked scores with (max, fac) in LDS; the output wavefront
// of g, one tile behind, rescales its accumulators and row sums by fac,
// forms P = exp(s - max) as fp16 (the C layout of S^T is the B operand layout
// of O^T += V^T P^T) and applies the tile with 16 MFMAs.  Each role needs
// about half the registers of one wavefront doing both, so the two share a
// SIMD and one's vector work runs under the other's matrix work.  The score
// side stages the K tiles and the output side the V^T tiles in the
// three-slot ring; one block barrier per tile orders all of it (every
// wavefront passes the same barriers).
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_attn_rs_kernel(PrefillArgs a) {
    __shared__ __align__(16) _Float16 ks[NKB][KT][KS2_LD];
    __shared__ __align__(16) _Float16 vs[NKB][256][VS2_LD];
    __shared__ __align__(16) f4 pss[2][4][4][64];     // masked scaled scores (slot, row group, quad, lane)
    __shared__ float2 pmf[2][4][64];                   // (reference max, rescale factor) per slot
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int wv = tid >> 6, lane = tid & 63;
    const int rg = wv & 3;           // row group
    const int t256 = tid & 255;      // staging thread within the role
    const int ln = lane & 31, hh = lane >> 5;
    const int n_rows = a.n_q * a.n_rep;
    const int row0 = (blockIdx.x * 4 + rg) * 32;
    const int split = blockIdx.z;
    const int k_lo = split * a.keys_per_split;
    const int k_hi = min(a.n_tot, k_lo + a.keys_per_split);
    const int H_q = a.h_kv * a.n_rep;
    const int r = row0 + ln;
    const bool r_ok = r < n_rows;
    const int jq = r_ok ? r / a.n_rep : 0;
    const int hq = h * a.n_rep + (r_ok ? r % a.n_rep : 0);
    const int b_last = min((int)blockIdx.x * 128 + 127, n_rows - 1);
    const int kt_hi = min(k_hi, block_key_end(a, blockIdx.x * 128, b_last));
    const int n_tiles = k_lo < kt_hi ? (kt_hi - k_lo + KT - 1) / KT : 0;
    const f32x16 zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    if (wv < 4) {
        // ================= score wavefront
        const RowKeys vis(a, r_ok, jq);
        h8 qb[16];
        {
            const __half* qrow = a.q + ((size_t)jq * H_q + hq) * 512;
#pragma unroll
            for (int st = 0; st < 16; st++) {
                const uint4 v = *reinterpret_cast<const uint4*>(qrow + 16 * st + 8 * hh);
                qb[st] = __builtin_bit_cast(h8, r_ok ? v : uint4{0u, 0u, 0u, 0u});
            }
        }
        // K tile staging: thread t -> key t / 8, 64 B at (t % 8) * 32 halves
        const int ld_key = t256 >> 3, ld_off = (t256 & 7) * 32;
        const __half* kg = a.k + (size_t)h * 256 + ld_off;
        uint4 pk[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pk[i] = uint4{0u, 0u, 0u, 0u};
        auto gload = [&](int k0) {
            const int key = min(k0 + ld_key, a.n_tot - 1);
            const uint4* ksrc = reinterpret_cast<const uint4*>(kg + (size_t)key * a.h_kv * 256);
#pragma unroll
            for (int i = 0; i < 4; i++) pk[i] = ksrc[i];
        };
        auto lstore = [&](int buf) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                *reinterpret_cast<uint4*>(&ks[buf][ld_key][ld_off + 8 * i]) = pk[i];
        };
        auto kread = [&](int buf, int half, h8 (&kop)[8]) {
#pragma unroll
            for (int i = 0; i < 8; i++)
                kop[i] = *reinterpret_cast<const h8*>(&ks[buf][ln][16 * (8 * half + i) + 8 * hh]);
        };
        if (n_tiles > 0) {
            gload(k_lo);
            lstore(0);
        }
        if (n_tiles > 1) {
            gload(k_lo + KT);
            lstore(1);
        }
        if (n_tiles > 2) gload(k_lo + 2 * KT);
        __syncthreads();  // prologue: K tiles 0, 1 and V^T tile 0 staged
        float m_ref = -INFINITY;
        f32x16 s2[2];
        {
            h8 kop[8];
            s2[0] = s2[1] = zero16;
#pragma unroll
            for (int half = 0; half < 2; half++) {
                kread(0, half, kop);
#pragma unroll
                for (int i = 0; i < 8; i++) s2[i & 1] = mfma3232(kop[i], qb[8 * half + i], s2[i & 1]);
            }
        }
        for (int t = 0; t < n_tiles; t++) {
            const int nxt = (t + 1) % NKB;
            const int k0 = k_lo + t * KT;
            float sc[16];
#pragma unroll
            for (int e = 0; e < 16; e++) sc[e] = s2[0][e] + s2[1][e];
            h8 kop[8];
            kread(nxt, 0, kop);
            // ---- S(t + 1), first half, under the mask and row maximum of tile t
            float lmax = -INFINITY;
            {
                const uint32_t mb = vis.tile(k0) >> (4 * hh);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    s2[i & 1] = mfma3232(kop[i], qb[i], i < 2 ? zero16 : s2[i & 1]);
#pragma unroll
                    for (int e = 2 * i; e < 2 * i + 2; e++) {  // key k0 + 8 (e / 4) + 4 hh + e % 4
                        sc[e] = (mb >> (8 * (e >> 2) + (e & 3))) & 1u ? sc[e] * a.sc : -INFINITY;
                        lmax = fmaxf(lmax, sc[e]);
                    }
                }
            }
            kread(nxt, 1, kop);
            // ---- raise the row's reference maximum only when needed; the
            // output wavefront rescales its accumulators and sums by fac
            float fac = 1.0f;
            if (__ballot(lmax > m_ref + GAP32) != 0ull) {
                const float rmax = fmaxf(lmax, __shfl_xor(lmax, 32, 64));
                const float m_new = fmaxf(m_ref, rmax);
                if (m_new > m_ref) {
                    fac = __expf(m_ref - m_new);  // 0 when m_ref = -inf (the sums are still 0)
                    m_ref = m_new;
                }
            }
            // ---- S(t + 1), second half; tile t's scores go to the output side
#pragma unroll
            for (int i = 0; i < 8; i++) s2[i & 1] = mfma3232(kop[i], qb[8 + i], s2[i & 1]);
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
                pss[t & 1][rg][q4][lane] = f4{sc[4 * q4], sc[4 * q4 + 1], sc[4 * q4 + 2], sc[4 * q4 + 3]};
            pmf[t & 1][rg][lane] = float2{m_ref, fac};
            // ---- stage K tile t + 2 (its slot last held tile t - 1), load t + 3
            if (t + 2 < n_tiles) {
                lstore((t + 2) % NKB);
                if (t + 3 < n_tiles) gload(k0 + 3 * KT);
            }
            __syncthreads();  // tile t
        }
        __syncthreads();  // the output side's last tile
    } else {
        // ================= output wavefront
        f32x16 acc[8];
#pragma unroll
        for (int t2 = 0; t2 < 8; t2++) acc[t2] = zero16;
        // V^T tile staging: thread t -> dim t, the tile's 32 keys (64 B)
        const __half* vg = a.vt + ((size_t)h * 256 + t256) * a.ld_vt;
        uint4 pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pv[i] = uint4{0u, 0u, 0u, 0u};
        auto gload = [&](int k0) {
            const uint4* vsrc = reinterpret_cast<const uint4*>(vg + k0);
#pragma unroll
            for (int i = 0; i < 4; i++) pv[i] = vsrc[i];
        };
        auto vmask = [](uint32_t w, int i, int nv) {
            return 2 * i + 1 < nv ? w : (2 * i < nv ? (w & 0xFFFFu) : 0u);
        };
        auto lstore = [&](int buf, int k0) {
            const int nv = a.n_tot - k0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                *reinterpret_cast<uint2*>(&vs[buf][t256][8 * i]) = uint2{pv[i].x, pv[i].y};
                *reinterpret_cast<uint2*>(&vs[buf][t256][8 * i + 4]) = uint2{pv[i].z, pv[i].w};
            }
            if (nv < KT) {  // the key space's last tile: V^T columns past n_tot cleared
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint4 v = pv[i];
                    *reinterpret_cast<uint2*>(&vs[buf][t256][8 * i]) =
                        uint2{vmask(v.x, 4 * i, nv), vmask(v.y, 4 * i + 1, nv)};
                    *reinterpret_cast<uint2*>(&vs[buf][t256][8 * i + 4]) =
                        uint2{vmask(v.z, 4 * i + 2, nv), vmask(v.w, 4 * i + 3, nv)};
                }
            }
        };
        // O^T += V^T P^T for tile u: 8 tiles of 32 dims x 2 K-steps of 16 keys
        float l_part = 0.0f, m_last = -INFINITY;
        auto pv_tile = [&](int u) {
            const int cur = u % NKB;
            // the tile's V^T operands first: their LDS latency runs under the
            // exponentials below
            h8 vop[2][8];
#pragma unroll
            for (int sp = 0; sp < 2; sp++)
#pragma unroll
                for (int t2 = 0; t2 < 8; t2++) {
                    const uint2 va = *reinterpret_cast<const uint2*>(&vs[cur][32 * t2 + ln][16 * sp + 4 * hh]);
                    const uint2 vb = *reinterpret_cast<const uint2*>(&vs[cur][32 * t2 + ln][16 * sp + 8 + 4 * hh]);
                    vop[sp][t2] = __builtin_bit_cast(h8, uint4{va.x, va.y, vb.x, vb.y});
                }
            const float2 mf = pmf[u & 1][rg][lane];
            const f4 s0 = pss[u & 1][rg][0][lane], s1 = pss[u & 1][rg][1][lane];
            const f4 s2v = pss[u & 1][rg][2][lane], s3 = pss[u & 1][rg][3][lane];
            const float sc[16] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3],
                                  s2v[0], s2v[1], s2v[2], s2v[3], s3[0], s3[1], s3[2], s3[3]};
            m_last = mf.x;
            if (__ballot(mf.y != 1.0f) != 0ull) {
#pragma unroll
                for (int t2 = 0; t2 < 8; t2++) acc[t2] *= mf.y;
                l_part *= mf.y;
            }
            float p[16];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                p[e] = sc[e] == -INFINITY ? 0.0f : __expf(sc[e] - mf.x);
                l_part += p[e];
            }
            h8 pbv[2];
#pragma unroll
            for (int sp = 0; sp < 2; sp++)
                pbv[sp] = __builtin_bit_cast(h8, uint4{pk_rne(p[8 * sp], p[8 * sp + 1]),
                                                       pk_rne(p[8 * sp + 2], p[8 * sp + 3]),
                                                       pk_rne(p[8 * sp + 4], p[8 * sp + 5]),
                                                       pk_rne(p[8 * sp + 6], p[8 * sp + 7])});
#pragma unroll
            for (int sp = 0; sp < 2; sp++)
#pragma unroll
                for (int t2 = 0; t2 < 8; t2++) acc[t2] = mfma3232(vop[sp][t2], pbv[sp], acc[t2]);
        };
        if (n_tiles > 0) {
            gload(k_lo);
            lstore(0, k_lo);
        }
        if (n_tiles > 1) gload(k_lo + KT);
        __syncthreads();  // prologue
        for (int t = 0; t < n_tiles; t++) {
            if (t >= 1) pv_tile(t - 1);
            // ---- stage V^T tile t + 1 (its slot last held tile t - 2), load t + 2
            if (t + 1 < n_tiles) {
                lstore((t + 1) % NKB, k_lo + (t + 1) * KT);
                if (t + 2 < n_tiles) gload(k_lo + (t + 2) * KT);
            }
            __syncthreads();  // tile t
        }
        if (n_tiles > 0) pv_tile(n_tiles - 1);
        __syncthreads();  // last tile applied
        const float l_row = l_part + __shfl_xor(l_part, 32, 64);
        // ---- partial triple of row ln (dims 32 t + 8 j + 4 hh + c)
        if (r_ok) {
            const float2 ml = float2{m_last, l_row};
            float* out = a.part + ((size_t)(jq * H_q + hq) * a.n_split + split) * 258;
            const bool empty = (ml.x == -INFINITY);
#pragma unroll
            for (int t2 = 0; t2 < 8; t2++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f4 v = f4{acc[t2][4 * j], acc[t2][4 * j + 1], acc[t2][4 * j + 2], acc[t2][4 * j + 3]};
                    *reinterpret_cast<f4*>(&out[32 * t2 + 8 * j + 4 * hh]) = empty ? f4{0.f, 0.f, 0.f, 0.f} : v;
                }
            if (hh == 0) {
                out[256] = empty ? -1e20f : ml.x;
                out[257] = empty ? 0.0f : ml.y;
            }
        }
    }
}

// Merge of the key splits, normalisation and gate: one wavefront per (query,
// head) row, lane l owning dims 4 l .. 4 l + 3; lane s < n_split holds split
// s's (m, l) pair.  Each group of up to 16 splits has every load in flight
// before the first is used (the first group's with the (m, l) loads, ahead of
// the maximum); the sums run in split order.
constexpr int MG = 16;  // splits per load group
__global__ __launch_bounds__(256) void prefill_merge_kernel(const float* __restrict__ part,
                                                            const __half* __restrict__ q_gate,
                                                            __half* __restrict__ out, int n_rows,
                                                            int n_split, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= n_rows) return;  // uniform per wavefront
    const float* base = part + (size_t)row * n_split * 258;
    float2 a[MG][2];
    auto load_group = [&](int s0) {
#pragma unroll
        for (int j = 0; j < MG; j++)
            if (s0 + j < n_split) {
                const float* pp = base + (size_t)(s0 + j) * 258 + 4 * lane;
                a[j][0] = *reinterpret_cast<const float2*>(pp);
                a[j][1] = *reinterpret_cast<const float2*>(pp + 2);
            }
    };
    load_group(0);  // in flight with the (m, l) pairs below
    float m = -1e30f, l = 0.0f;
    if (lane < n_split) {
        const float2 ml = *reinterpret_cast<const float2*>(base + (size_t)lane * 258 + 256);
        m = ml.x;
        l = ml.y;
    }
    float M = m;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    const float w = lane < n_split ? __expf(m - M) : 0.0f;
    const float lw = l * w;
    float num[4] = {0.f, 0.f, 0.f, 0.f}, den = 0.0f;
    for (int s0 = 0; s0 < n_split; s0 += MG) {
        if (s0 > 0) load_group(s0);
#pragma unroll
        for (int j = 0; j < MG; j++)
            if (s0 + j < n_split) {
                const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s0 + j));
                num[0] = fmaf(a[j][0].x, ws, num[0]);
                num[1] = fmaf(a[j][0].y, ws, num[1]);
                num[2] = fmaf(a[j][1].x, ws, num[2]);
                num[3] = fmaf(a[j][1].y, ws, num[3]);
                den += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lw), s0 + j));
            }
    }
    const uint2 gw = *reinterpret_cast<const uint2*>(q_gate + (size_t)row * 512 + 256 + 4 * lane);
    const h4 g = __builtin_bit_cast(h4, gw);
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; c++)
        o[c] = num[c] / (den + eps) * (1.0f / (1.0f + expf(-(float)g[c])));
    *reinterpret_cast<uint2*>(out + (size_t)row * 256 + 4 * lane) =
        uint2{pk_rne(o[0], o[1]), pk_rne(o[2], o[3])};
}

}  // namespace pf

hipError_t launch_prefill_merge(const float* part, const __half* q_gate, __half* out, int n_rows,
                                int n_split, float eps, hipStream_t st) {
    hipLaunchKernelGGL(pf::prefill_merge_kernel, dim3((n_rows + 3) / 4), dim3(256), 0, st, part,
                       q_gate, out, n_rows, n_split, eps);
    return hipGetLastError();
}

hipError_t launch_decompress(const DecompArgs& a, hipStream_t st) {
    if (a.n_tok <= 0) return hipSuccess;
    hipLaunchKernelGGL(pf::decompress_kernel, dim3((a.n_tok + pf::TOK_BLK - 1) / pf::TOK_BLK, a.h_kv),
                       dim3(pf::BLK_THR), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_decompress_gather(const DecompArgs& d, const GatherArgs& g, hipStream_t st) {
    const int side = g.src_k && g.side_n > 0 ? 1 : 0;
    const int n_g = std::max(g.n, side ? g.side_n : 0);
    if (d.n_tok <= 0) return launch_ring_gather(g, st);
    if (n_g <= 0) return launch_decompress(d, st);
    const int nx_d = (d.n_tok + pf::TOK_BLK - 1) / pf::TOK_BLK;
    const int nx_g = (n_g + pf::TOK_BLK - 1) / pf::TOK_BLK;
    hipLaunchKernelGGL(pf::decompress_gather_kernel,
                       dim3(nx_d * d.h_kv + nx_g * g.h_kv * (1 + side)), dim3(pf::BLK_THR), 0, st,
                       d, g, nx_d, nx_g);
    return hipGetLastError();
}

hipError_t launch_compress_decode(const CompressJob& k, const CompressJob& v, const DecompArgs& d,
                                  const GatherArgs* g, hipStream_t st) {
    // the decode covers exactly the compressed rows: token t, KV head h is row t h_kv + h
    if (k.n != v.n || d.n_tok * d.h_kv != k.n || d.tok0 != d.key0 || d.start_pos != 0)
        return hipErrorInvalidValue;
    const int nb_k = (k.n + 3) / 4;
    int nx_g = 0, planes = 0;
    GatherArgs ga{};
    if (g) {
        const int side = g->src_k && g->side_n > 0 ? 1 : 0;
        const int n_g = std::max(g->n, side ? g->side_n : 0);
        if (n_g > 0) {
            nx_g = (n_g + pf::TOK_BLK - 1) / pf::TOK_BLK;
            planes = 1 + side;
            ga = *g;
        }
    }
    hipLaunchKernelGGL(pf::compress_decode_kernel, dim3(v.n + nb_k + nx_g * ga.h_kv * planes),
                       dim3(pf::BLK_THR), 0, st, k, v, d, ga, nb_k, nx_g);
    return hipGetLastError();
}

hipError_t launch_ring_gather(const GatherArgs& a, hipStream_t st) {
    const int side = a.src_k && a.side_n > 0 ? 1 : 0;
    const int n = std::max(a.n, side ? a.side_n : 0);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(pf::ring_gather_kernel,
                       dim3((n + pf::TOK_BLK - 1) / pf::TOK_BLK, a.h_kv, 1 + side),
                       dim3(pf::BLK_THR), 0, st, a);
    return hipGetLastError();
}

namespace {
// Few query rows (a handful of queries, e.g. the one after a compression
// event): the 16-row kernel, two blocks per CU (more, shorter splits); many:
// the role-specialised 32-row kernel (half the LDS operand traffic per flop).
bool few_rows(int n_rows) { return n_rows <= 128; }
}  // namespace

int prefill_splits(int n_q, int n_rep, int h_kv, int n_k, int* keys_per_split) {
    // Blocks that run at once: 2 per CU for the 16-row kernel (72 KB of LDS
    // each), 1 for the 32-row kernel (142 KB).  The split count fills that
    // many slots in one round: a few blocks past a round cost a whole round.
    const int n_cu = device_cu_count();
    const int n_rows = n_q * n_rep;
    const bool few = few_rows(n_rows);
    const int slots = few ? 2 * n_cu : n_cu;
    const int blocks = (few ? ((n_rows + 15) / 16 + 3) / 4 : (n_rows + 127) / 128) * h_kv;
    int ns = slots / blocks;
    ns = std::max(1, std::min(ns, 64));
    int per = (n_k + ns - 1) / ns;
    per = (per + pf::KT - 1) / pf::KT * pf::KT;
    ns = (n_k + per - 1) / per;
    *keys_per_split = per;
    return std::max(ns, 1);
}

hipError_t launch_prefill_attn(const PrefillArgs& a, hipStream_t st) {
    const int n_rows = a.n_q * a.n_rep;
    if (few_rows(n_rows)) {
        const int mtiles = (n_rows + 15) / 16;
        hipLaunchKernelGGL(pf::prefill_attn_kernel, dim3((mtiles + 3) / 4, a.h_kv, a.n_split),
                           dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(pf::prefill_attn_rs_kernel, dim3((n_rows + 127) / 128, a.h_kv, a.n_split),
                           dim3(512), 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace khq
