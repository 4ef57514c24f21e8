// khq_internal.h -- kernel argument blocks and launch helpers shared by the
// kernels (khq_kernels.hip) and the C ABI layer (khq_capi.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <atomic>

namespace khq {

// Compressed-region work: token range [0, c_len) of KV head blockIdx.y cut
// into n_parts parts; the partial triple of query qid, part i lands at
// part[(qid * part_stride + part_offset + i) * 258].
struct AttnArgs {
    const __half* q;  // q_gate [H_q][512]
    const uint8_t* kpay;
    const uint8_t* vpay;
    const uint8_t* vsm;
    const uint32_t* kmask;
    const __half* knorm;
    const __half* krn;
    const __half* vnorm;
    const __half* vrn;
    const __half* cents_k;
    const __half* cents_v;
    const __half* vq;
    const __half* rotor_k;
    const __half* rotor_v;
    const __half* dk;
    const __half* dv;
    float* part;
    int c_len, h_kv, L_q, start_pos, n_parts, part_stride, part_offset;
    float sc, a_k, a_v, rope_base;
    // Optional raw ring window, computed by one extra block of the
    // wavefront-specialised kernel into partial part_offset + n_chunks
    // (win_len = 0: none).
    const __half* ring_k;
    const __half* ring_v;
    int win_start, win_len, ring_cap;
    int win_blocks;  // window blocks after the chunks: 4 (one per KV head) or 1 (all heads)
    int chunk_tiles;  // batched launch: tiles per compressed chunk of this sequence
    // Bound of the key / value hand-off waits of the wavefront-specialised
    // kernel, in sleeps (set by the launchers; a test knob may lower it).
    int spin_limit;
    // Reference split partition (wavefront-specialised kernel): split_per > 0
    // cuts [0, c_len) into splits of split_per tokens, each into split_subs
    // chunks of tiles_per_chunk tiles; chunk = split * split_subs + sub.
    // split_per = 0: chunk i covers tiles [i * tiles_per_chunk, + tiles_per_chunk).
    int split_per, split_subs;
    // RoPE table of the wavefront-specialised kernel, [lane group g][3][u]:
    // freq of dim pair m = 16 (u / 4) + 4 g + u % 4, cos and sin of 16 freq
    // (filled by the launchers from rope_base).
    float rope_tab[96];
};

// fp16 ring-window work, same partial layout (query = head).
struct WinArgs {
    const __half* q;
    const __half* ring_k;
    const __half* ring_v;
    float* part;
    int win_start, win_len, ring_cap, h_kv, n_parts, part_stride, part_offset;
    float sc;
};

// Window attention + merge with compressed partials + gate (fused step tail).
// Compressed partial i of query head h at part[(h * part_stride + i) * 258].
struct FinishArgs {
    const float* part;
    int n_parts, part_stride;
    const __half* q;  // q_gate [H_q][512]
    const __half* ring_k;
    const __half* ring_v;
    int win_start, win_len, ring_cap, h_kv, n_rep;
    float sc, eps;
    __half* out;  // [H_q][256]
};
hipError_t launch_step_finish(const FinishArgs& a, int H_q, hipStream_t st);
// n_seq sequences, args a device array; the window must already be a part
// (win_len = 0 in every FinishArgs).
// Copies bytes (a multiple of 16) from pinned host memory to device memory
// with a one-block kernel on st.
hipError_t launch_meta_upload(const void* host_src, void* dst, size_t bytes, hipStream_t st);
hipError_t launch_step_finish_batched(const FinishArgs* args, int n_seq, int H_q,
                                      hipStream_t st);

// One compressor job (the arguments of launch_compress without is_v).
struct CompressJob {
    const __half* x;
    const __half* d_vec;
    const __half* rotor;
    const __half* cents;
    const __half* vq;
    uint32_t* out_mask;
    __half* out_norms;
    __half* out_rn;
    uint8_t* out_pay;
    uint8_t* out_sm;
    int n;
    float ts, alpha;
};
// The K and V jobs of one compression event in one launch.
hipError_t launch_compress_pair(const CompressJob& k, const CompressJob& v, hipStream_t st);
hipError_t launch_compress(const __half* x, const __half* d_vec, const __half* rotor,
                           const __half* cents, const __half* vq, uint32_t* out_mask,
                           __half* out_norms, __half* out_rn, uint8_t* out_pay,
                           uint8_t* out_sm, int n, float ts, float alpha, int is_v,
                           hipStream_t st);
hipError_t launch_attn_parts(const AttnArgs& a, int n_rep, dim3 grid, hipStream_t st);
hipError_t launch_window_parts(const WinArgs& a, int n_rep, dim3 grid, hipStream_t st);
hipError_t launch_lse_reduce(const float* part, float* out, int n_q, int n_parts,
                             hipStream_t st);
hipError_t launch_combine_gate(const float* part, const __half* q_gate, __half* out, int H_q,
                               int n_parts, float eps, hipStream_t st);
hipError_t launch_merge_gate(const float* ac, const float* aw, const __half* qg, __half* out,
                             int H_q, int D, int has_w, hipStream_t st);
hipError_t launch_gather_q(const __half* qg, __half* qo, int H_q, int D, hipStream_t st);
hipError_t launch_ring_write(__half* rk, __half* rv, __half* ru, const __half* k,
                             const __half* v, const __half* ku, int kv, hipStream_t st);
hipError_t launch_partial_rope(__half* vec, int num_heads, int head_dim, int rotary_dim, int pos,
                               float theta, int stride, hipStream_t st);

// Compressed-region kernel for H_kv = 4, n_rep = 6, L_q = 1 (wavefront-
// specialised, 512 threads per block): one block per chunk of
// tiles_per_chunk 16-token tiles; partial index = part_offset + chunk.
int attn_ws_tiles_per_chunk(int c_len, int* n_chunks);
// Device fault word of the wavefront-specialised kernel (nonzero after a
// hand-off wait gave up), read with a synchronous copy; clear resets it.
hipError_t fault_status(int* out, int clear);
// Hand-off wait bound used by the launchers (default 2^20 sleeps).
extern std::atomic<int> g_spin_limit;
size_t attn_ws_smem_bytes();
// Fills a.rope_tab from a.rope_base (host).
void fill_rope_table(AttnArgs& a);
hipError_t launch_attn_ws(const AttnArgs& a, int tiles_per_chunk, int n_chunks,
                          hipStream_t st);
// Batched: args[seq] (device) with n_parts = that sequence's chunk count and
// its window fields; map[b] = (seq, chunk) for each of n_blocks blocks (chunk
// == n_parts: the sequence's window block).
hipError_t launch_attn_ws_batched(const AttnArgs* args, const int2* map, int n_blocks,
                                  hipStream_t st);

// Head RMSNorm + unroped capture + partial RoPE + ring writes of one token
// (D = 256, rot <= 64): q_gate [H_q][512] and k [H_kv][256] in place.
struct NormRopeArgs {
    __half* q_gate;
    __half* k;
    const __half* v;
    const float* q_w;  // [256] or NULL
    const float* k_w;  // [256] or NULL
    __half* ring_k;
    __half* ring_v;
    __half* ring_u;
    int H_q, H_kv, slot, pos, rot;
    float eps, theta;
};
hipError_t launch_norm_rope(const NormRopeArgs& a, hipStream_t st);

// ---- chunked prefill (khq_prefill.hip)
// Compressed rows [tok0, tok0 + n_tok) of every KV head -> dense fp16 roped K
// rows out_k[(key0 + t) * h_kv + h][256] and V^T out_vt[h][256][ld_vt]
// columns key0 + t (ld_vt >= key0 + n_tok rounded up to 64, multiple of 8).
struct DecompArgs {
    const uint8_t* kpay;
    const uint8_t* vpay;
    const uint8_t* vsm;
    const uint32_t* kmask;
    const __half* knorm;
    const __half* krn;
    const __half* vnorm;
    const __half* vrn;
    const __half* cents_k;
    const __half* cents_v;
    const __half* vq;
    const __half* rotor_k;
    const __half* rotor_v;
    const __half* dk;
    const __half* dv;
    __half* out_k;
    __half* out_vt;
    int h_kv, tok0, n_tok, start_pos, key0, ld_vt;
    float a_k, a_v, rope_base;
};
// Ring slots (win_start + t) % ring_cap, t < n -> the same key layout at key0 + t.
struct GatherArgs {
    const __half* ring_k;
    const __half* ring_v;
    __half* out_k;
    __half* out_vt;
    int h_kv, win_start, n, ring_cap, key0, ld_vt;
    // Chunk mode (src_k != null): token t comes from src_k / src_v / src_u
    // rows [t][h_kv][256] instead of the ring, and is also written to ring
    // slot (win_start + t) % ring_cap of wr_k / wr_v / wr_u (wr_u optional).
    const __half* src_k;
    const __half* src_v;
    const __half* src_u;
    __half* wr_k;
    __half* wr_v;
    __half* wr_u;
    // Second job (grid z = 1, chunk mode only): side_n tokens whose first
    // side_from_src come from ring slots (side_start + t) % ring_cap and the
    // rest from src rows t - side_from_src, written to keys side_key0 + t.
    int side_n, side_start, side_from_src, side_key0;
};
// n_q queries (q_gate rows [n_q][H_q][512]) over dense keys [0, n_k); query j
// sees keys [0, min(n_k, vis0 + j)).  Partial triple of (query j, head hq,
// split s) at part[((j * H_q + hq) * n_split + s) * 258].
struct PrefillArgs {
    const __half* q;
    const __half* k;
    const __half* vt;
    float* part;
    int ld_vt, n_k, n_q, vis0, h_kv, n_rep, n_split, keys_per_split;
    float sc;
    // Keys are indices [0, n_tot), n_tot >= n_k.  Queries j < q_b (the run
    // before a compression event) lose [hole_lo, hole_hi) and see key
    // ex_lo + i for position hole_lo + i (when that position is below their
    // causal limit) instead: the raw copies of the compressed chunk, placed
    // past n_k, while the main key space holds its decoded rows for the
    // queries after the event.  q_b = 0: no such run.
    int n_tot, q_b, hole_lo, hole_hi, ex_lo, ex_hi;
};
hipError_t launch_decompress(const DecompArgs& a, hipStream_t st);
hipError_t launch_ring_gather(const GatherArgs& a, hipStream_t st);
// A decode and a gather whose outputs are disjoint, in one launch.
hipError_t launch_decompress_gather(const DecompArgs& d, const GatherArgs& g, hipStream_t st);
// A compression event (k, v: rows (token, KV head) of the chunk), the decode
// of those rows (d: tok0 = key0, n_tok tokens, start_pos 0) and an optional
// independent gather (chunk append or raw copy) in one launch.
hipError_t launch_compress_decode(const CompressJob& k, const CompressJob& v, const DecompArgs& d,
                                  const GatherArgs* g, hipStream_t st);
int prefill_splits(int n_q, int n_rep, int h_kv, int n_k, int* keys_per_split);
hipError_t launch_prefill_attn(const PrefillArgs& a, hipStream_t st);
// Prefill attention plus merge and gate through the shared workspace; the
// hole / extra ranges as in PrefillArgs (all zero: plain causal prefill);
// merge = false: the attention launch alone (partials left in the workspace).
int prefill_attn_run(const __half* q_gate, const __half* k, const __half* vt, int ld_vt, int n_k,
                     int n_q, int vis0, int H_q, int H_kv, float scale, __half* out,
                     hipStream_t stream, int q_b, int hole_lo, int hole_hi, int ex_lo, int ex_hi,
                     bool merge = true);
// Merge of n_split partial triples per row, / (den + eps), sigmoid gate from
// q_gate row r (f16 [r][512], gate at 256..511): out f16 [r][256].
hipError_t launch_prefill_merge(const float* part, const __half* q_gate, __half* out, int n_rows,
                                int n_split, float eps, hipStream_t st);

// Per-device launch set-up, cached per device index under a lock (a process
// may drive several GPUs from several threads): the CU count of the current
// device, and the dynamic-LDS limit of a kernel raised to `bytes` on the
// current device (once per (kernel, device)).
int device_cu_count();
hipError_t ensure_dynamic_lds(const void* kernel, int bytes);

}  // namespace khq
