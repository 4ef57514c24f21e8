/*
 * khq.h -- C ABI of libkhq_hip.so, the MI355X (gfx950) KHQ decode-attention
 * library.
 *
 * The first five entry points are drop-ins for the extern "C" launchers of
 * oki-abrian/bonsai-mojo-1bit-optimization-t4-cuda's libbonsai_qmv_sm75.so:
 * same names, same argument order and meaning, same return codes
 * (0 = ok, -100 = bad shape, -101 = split-K without a partial buffer,
 * otherwise a positive hipError_t), with hipStream_t in place of
 * cudaStream_t.  All pointers are device pointers owned by the caller.
 * Launches are asynchronous on `stream` (NULL = the null stream).
 *
 * Layouts (row r = token * H_kv + kv_head, 220 B per row in total):
 *   k_mask  u32[r][16]   2-bit codes, dim i at word i/16 bits 2*(i%16)
 *   k_pay   u8 [r][40]   c_base_mult*1000 (u32), 50 residual nibbles,
 *                        50 sign bits, 0x02 marker
 *   k_norm, k_rn  f16[r] norm, residual scale
 *   v_pay   u8 [r][104]  64 x 12-bit patch fields + 2 words of VQ bit 7
 *   v_norm, v_rn  f16[r] norm, energy correction
 *   v_sm    u8 [r][4]    f32 max |dim-3 residual|
 *   q_gate  f16[H_q][2*256]  q at 0..255, gate at 256..511 (per head)
 *   ring_k/ring_v f16[ring_cap][H_kv][256]
 *   out_attn f32[queries][258]  unnormalised (acc[256], max, sum_exp)
 */
#ifndef KHQ_H
#define KHQ_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces launch_khq_compress_fp16, ref:src/csrc/qmv_sm75_kernel.cu:4279-4310.
 * Compresses n rows of x (f16 [n][256]).  is_v=0: K branch (writes mask,
 * norms, residual scale, 40-B payload, shared meta = 0).  is_v=1: V branch
 * (writes norms, energy, 104-B payload, shared meta = max residual; the mask
 * is not touched).  Codes are bit-exact with the CPU restatement. */
int launch_khq_compress_fp16(const void* x, const void* d_vec, const void* rotor,
                             const void* centroids, const void* vq_centroids,
                             void* out_mask, void* out_norms, void* out_r_norms,
                             void* out_payload, void* out_shared_meta, int n, int d,
                             float threshold_scale, float alpha, int is_v,
                             hipStream_t stream);

/* Replaces launch_khq_attn_fp16, ref:.cu:4314-4375.  Attention of
 * num_queries = num_heads * L_q queries over compressed tokens [0, c_len),
 * RoPE on dims 0..63 at absolute position start_pos + s.  Writes the
 * unnormalised triple to out_attn.  num_splits > 1 (out_partial required,
 * else -101) selects the reference's partition: split i covers tokens
 * [i * per, (i + 1) * per), per = ceil(s_limit / num_splits), and its triple
 * is written to out_partial f32 [num_queries][num_splits][258] (empty splits:
 * acc 0, max -1e20, sum 0); out_attn is their logsumexp merge.  Internally
 * each split may be cut further (library workspace) and merged into its
 * triple first.  num_splits <= 1: the library's own partition, out_partial
 * untouched.  stride_s is unused, as in the reference. */
int launch_khq_attn_fp16(const void* q, const void* k_payload, const void* v_payload,
                         const void* v_shared_meta, const void* k_mask,
                         const void* k_norms, const void* k_r_norms, const void* v_norms,
                         const void* v_r_norms, const void* centroids_k,
                         const void* centroids_v, const void* vq_centroids,
                         const void* k_rotor, const void* v_rotor, const void* d_vec_k,
                         const void* d_vec_v, void* out_attn, void* out_partial,
                         int num_queries, int num_heads, int L_q, int c_len,
                         int stride_s, int n_rep, float scale, float alpha_k,
                         float alpha_v, float rope_base, int start_pos,
                         int num_splits, hipStream_t stream);

/* The split-K merge launch_khq_attn_fp16 issues when num_splits > 1, on its
 * own (the reference launches khq_attn_reduce_kernel, ref:.cu:1836-1877,
 * only inside launch_khq_attn_fp16, :4366-4373): logsumexp merge of
 * partial f32 [num_queries][num_splits][258] into out_attn f32
 * [num_queries][258].  Empty splits (max -1e20, sum 0) weigh nothing. */
int khq_attn_reduce_f32(const void* partial, void* out_attn, int num_queries, int num_splits,
                        hipStream_t stream);

/* Replaces launch_khq_window_attn_fp16, ref:.cu:4378-4396.  fp16 attention of
 * H_q heads over ring slots (win_start + s) % ring_cap, s < win_len (K already
 * roped).  Unnormalised triple into out_attn f32[H_q][258].  Beyond the
 * reference it returns -100 for d != 256, H_q % H_kv != 0, H_q/H_kv > 8 or
 * win_len > ring_cap instead of reading stale slots. */
int launch_khq_window_attn_fp16(const void* q, const void* ring_k, const void* ring_v,
                                void* out_attn, int win_start, int win_len, int ring_cap,
                                int H_q, int H_kv, int d, float scale, hipStream_t stream);

/* Replaces launch_khq_gather_q_fp16, ref:.cu:4399-4411. */
int launch_khq_gather_q_fp16(const void* q_gate, void* q_out, int H_q, int d,
                             hipStream_t stream);

/* Replaces launch_khq_merge_gate_fp16, ref:.cu:4414-4429.  Logsumexp merge of
 * the compressed and window triples (has_w = 0: attn_c only), divide by
 * (den + 1e-8), times sigmoid(gate), f16 out [H_q][d]. */
int launch_khq_merge_gate_fp16(const void* attn_c, const void* attn_w, const void* q_gate,
                               void* out, int H_q, int d, int has_w, hipStream_t stream);

/* ---- helpers the reference implements as Mojo GPU kernels ---- */

/* Replaces khq_ring_dual_sm75_gpu + copy_vec_sm75_gpu
 * (ref:src/kernels/elementwise_sm75.mojo:277-312, called from
 * ref:src/khq/runtime.mojo:432-451,486-488): one launch copies one token's
 * roped K, V and unroped K into ring slot `slot` of ring_k, ring_v, ring_u.
 * Any of the three (destination, source) pairs may be (NULL, NULL), not all.
 * kv = H_kv * 256 halves per tensor. */
int launch_khq_ring_write_fp16(void* ring_k, void* ring_v, void* ring_u,
                               const void* k_roped, const void* v, const void* k_unroped,
                               int slot, int kv, hipStream_t stream);

/* Replaces partial_rope_sm75_gpu (ref:elementwise_sm75.mojo:1023-1061):
 * half-split RoPE on dims 0..rotary_dim-1 of each head, in place, heads
 * `stride` halves apart (0 = head_dim). */
int launch_khq_partial_rope_fp16(void* vec, int num_heads, int head_dim, int rotary_dim,
                                 int pos, float theta_base, int stride, hipStream_t stream);

/* Replaces gqa_attention_sm75_gpu (ref:elementwise_sm75.mojo:1091-1231), the
 * uncompressed fp16 baseline: GQA softmax attention of q_gate over
 * k_cache/v_cache f16 [seq][H_kv][256] (positions 0..seq_len-1), softmax
 * denominator Z + 1e-9, times sigmoid(gate), f16 out [H_q][256]. */
int launch_khq_gqa_attn_fp16(const void* q_gate, const void* k_cache, const void* v_cache,
                             void* out, int seq_len, int H_q, int H_kv, int head_dim,
                             float scale, hipStream_t stream);

/* ---- fused layer step (no reference counterpart: the reference issues
 * launch_khq_attn_fp16 + launch_khq_window_attn_fp16 +
 * launch_khq_merge_gate_fp16 from ref:src/khq/runtime.mojo:554-613) ----
 * Both regions in one pass: compressed tokens [0, c_len) (c_len may be 0) and
 * ring window slots (win_start + s) % ring_cap, s < win_len (win_len may be
 * 0), merged by logsumexp, divided by (den + 1e-8), gated, f16 out [H_q][256].
 * Returns -100 if both regions are empty. */
int khq_attn_step_fp16(const void* q_gate, const void* k_payload, const void* v_payload,
                       const void* v_shared_meta, const void* k_mask, const void* k_norms,
                       const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                       const void* centroids_k, const void* centroids_v,
                       const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                       const void* d_vec_k, const void* d_vec_v, const void* ring_k,
                       const void* ring_v, void* out, int H_q, int H_kv, int c_len,
                       int win_start, int win_len, int ring_cap, float scale,
                       float alpha_k, float alpha_v, float rope_base, hipStream_t stream);

/* No counterpart in the reference: khq_attn_step_fp16 for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results; its
 * split partials live in a fixed 8 MiB device array of the library (one per
 * GPU, held until the process ends) instead of the growable workspace, so it
 * calls no hipMalloc / hipFree.  Returns -103 when the partials would exceed
 * that array (H_q * parts * 258 floats; H_q 24 fits at any context).  Calls
 * that overlap on one GPU share the array and race. */
int khq_attn_step_noalloc_fp16(const void* q_gate, const void* k_payload,
                               const void* v_payload, const void* v_shared_meta,
                               const void* k_mask, const void* k_norms, const void* k_r_norms,
                               const void* v_norms, const void* v_r_norms,
                               const void* centroids_k, const void* centroids_v,
                               const void* vq_centroids, const void* k_rotor,
                               const void* v_rotor, const void* d_vec_k, const void* d_vec_v,
                               const void* ring_k, const void* ring_v, void* out, int H_q,
                               int H_kv, int c_len, int win_start, int win_len, int ring_cap,
                               float scale, float alpha_k, float alpha_v, float rope_base,
                               hipStream_t stream);

/* ---- batched decode (no reference counterpart: the reference decodes one
 * sequence at a time through khq_step, ref:src/khq/runtime.mojo:454-613) ----
 * n_seq independent sequences of one layer (shared constant tensors), one
 * query token each, each with its own payload, ring, c_len and window, as in
 * khq_attn_step_fp16.  seqs is a host array.  With the 24/4/256 shape one
 * launch covers every sequence's compressed chunks and windows and a second
 * one merges and gates; other shapes run one fused step per sequence. */
typedef struct khq_seq {
    const void* q_gate;  /* f16 [H_q][512] */
    const void* k_payload;
    const void* v_payload;
    const void* v_shared_meta;
    const void* k_mask;
    const void* k_norms;
    const void* k_r_norms;
    const void* v_norms;
    const void* v_r_norms;
    const void* ring_k;  /* f16 [ring_cap][H_kv][256] */
    const void* ring_v;
    void* out;           /* f16 [H_q][256] */
    int c_len, win_start, win_len, ring_cap;
} khq_seq;
/* Decode of compressed rows to dense fp16 (counterpart of the reference's
 * calibration decoders cal_decompress_k / cal_decompress_v,
 * ref:src/csrc/qmv_sm75_kernel.cu:2722-3024, with the attention kernel's
 * decode and RoPE, :1608-1699, :1739-1762, :1776-1826): tokens [tok0, tok0 +
 * n_tok) of every KV head -> out_k f16 [key0 + t][H_kv][256] (roped at
 * position start_pos + tok0 + t) and out_vt f16 [H_kv][256][ld_vt] columns
 * key0 + t.  key0 and ld_vt: multiples of 8, ld_vt >= key0 + n_tok rounded up
 * to 64. */
int khq_decompress_fp16(const void* k_payload, const void* v_payload, const void* v_shared_meta,
                        const void* k_mask, const void* k_norms, const void* k_r_norms,
                        const void* v_norms, const void* v_r_norms, const void* centroids_k,
                        const void* centroids_v, const void* vq_centroids, const void* k_rotor,
                        const void* v_rotor, const void* d_vec_k, const void* d_vec_v, int H_kv,
                        int tok0, int n_tok, int start_pos, float alpha_k, float alpha_v,
                        float rope_base, void* out_k, int key0, void* out_vt, int ld_vt,
                        hipStream_t stream);
/* Causal attention of n_q query tokens over dense fp16 keys (no reference
 * counterpart; the multi-query form of khq_attn_step_fp16's two regions):
 * k f16 [n_k][H_kv][256], vt f16 [H_kv][256][ld_vt]; query j (q_gate row j,
 * f16 [n_q][H_q][512]) sees keys [0, min(n_k, vis0 + j)).  out f16
 * [n_q][H_q][256] = softmax-weighted V / (den + 1e-8) * sigmoid(gate), the
 * merge_gate convention.  ld_vt: a multiple of 8 and at least n_k rounded up
 * to 32 (V^T is read in 32-key tiles); smaller returns -100. */
int khq_prefill_attn_fp16(const void* q_gate, const void* k, const void* vt, int ld_vt, int n_k,
                          int n_q, int vis0, int H_q, int H_kv, float scale, void* out,
                          hipStream_t stream);
/* Profiling entry (no reference counterpart): launches only the attention
 * kernel of khq_prefill_attn_fp16 (split partials into the library
 * workspace, nothing merged), so its duration can be timed on its own. */
int khq_prefill_attn_partials_fp16(const void* q_gate, const void* k, const void* vt, int ld_vt,
                                   int n_k, int n_q, int vis0, int H_q, int H_kv, float scale,
                                   hipStream_t stream);

/* khq_attn_step_batched_fp16 copies its per-sequence arguments from host
 * staging memory on every call, so it returns -105 on a stream under HIP
 * graph capture (a captured copy would replay stale arguments). */
int khq_attn_step_batched_fp16(const khq_seq* seqs, int n_seq, const void* centroids_k,
                               const void* centroids_v, const void* vq_centroids,
                               const void* k_rotor, const void* v_rotor, const void* d_vec_k,
                               const void* d_vec_v, int H_q, int H_kv, float scale,
                               float alpha_k, float alpha_v, float rope_base, hipStream_t stream);

/* Profiling entry (no reference counterpart): launches only the
 * compressed-region kernel of khq_attn_step_fp16 (partials into the library
 * workspace, nothing merged), so its duration can be timed on its own. */
int khq_attn_partials_fp16(const void* q_gate, const void* k_payload, const void* v_payload,
                           const void* v_shared_meta, const void* k_mask, const void* k_norms,
                           const void* k_r_norms, const void* v_norms, const void* v_r_norms,
                           const void* centroids_k, const void* centroids_v,
                           const void* vq_centroids, const void* k_rotor, const void* v_rotor,
                           const void* d_vec_k, const void* d_vec_v, int H_q, int H_kv,
                           int c_len, float scale, float alpha_k, float alpha_v,
                           float rope_base, hipStream_t stream);

/* Number of compressed-region token parts the library uses for c_len
 * (exposed for tests and the benchmark). */
int khq_attn_parts(int c_len);

/* Kernel choice for the compressed region (no reference counterpart; a
 * test and benchmark knob): 0 = automatic (matrix-core kernel for H_kv 4 /
 * n_rep 6 / L_q 1, portable kernel otherwise), 1 = portable kernel always.
 * Process-wide; returns -100 for other values. */
int khq_select_kernel(int which);

/* Fault word of the compressed-region kernel on the current device (no
 * reference counterpart).  The kernel's key and value wavefronts hand tiles
 * over through bounded waits; a wait that gives up makes that block write NaN
 * maxima into its partials (so the merged output is NaN, never silently
 * wrong) and sets bit 0 of this word.  Synchronous (it waits for the device's
 * queued work); clear = 1 resets the word after reading it. */
int khq_fault_status(int* flags, int clear);

/* Test knob (no reference counterpart): bound of those hand-off waits in
 * sleeps, process-wide; 0 restores the default (2^20). */
int khq_set_spin_limit(int sleeps);

/* Grows the library's device workspace (split partials) to at least `bytes`
 * on the current device.  Every launcher grows it on demand; call this first
 * when the launches will be captured into a HIP graph. */
int khq_workspace_reserve(size_t bytes);

/* Library version string. */
const char* khq_version(void);

/* ---- per-layer runtime (replaces KhqLayer / khq_init_layer /
 * khq_capture_unroped / khq_step, ref:src/khq/runtime.mojo:77-152,395-613;
 * the reference keeps this state in Mojo host structs) ----
 * A layer owns its 256-slot rings (roped K, V, unroped K), the packed payload
 * for cap_tokens tokens and its scratch; the constant tensors (centroids,
 * VQ codebook, rotors, d vectors, fp16 device buffers in the KHQK layouts)
 * stay owned by the caller and must outlive the layer.  splits follows
 * BONSAI_KHQ_SPLITS (clamped to [1, 64]) and only matters when fused = 0
 * (the reference's attn + window + merge launch sequence); fused = 1 issues
 * khq_attn_step_fp16.  Returns NULL on bad arguments or allocation failure. */
typedef struct khq_layer khq_layer;
khq_layer* khq_layer_create(int H_q, int H_kv, int cap_tokens, const void* centroids_k,
                            const void* centroids_v, const void* vq_centroids,
                            const void* k_rotor, const void* v_rotor, const void* d_vec_k,
                            const void* d_vec_v, float ts_k, float alpha_k, float ts_v,
                            float alpha_v, float rope_base, int splits, int fused);
void khq_layer_destroy(khq_layer* layer);
/* boundary = write_pos = 0 (the reference has none, README:260). */
int khq_layer_reset(khq_layer* layer);
int khq_layer_state(const khq_layer* layer, int* boundary, int* write_pos, int* n_events);
/* Device pointers of kmask, kpay, knorm, krn, vpay, vnorm, vrn, vsm, ring_k,
 * ring_v, ring_u (11 entries), for inspection. */
int khq_layer_payload(const khq_layer* layer, void** ptrs);
/* The prefill path's dense key space, for inspection: roped K rows
 * [keys][H_kv][256] (*k), V^T [H_kv][256][*ld_vt] (*vt), rows [0, *n_decoded)
 * decoded from the compressed region (null pointers before the first
 * prefill).  No counterpart in the reference (its prefill steps token by
 * token). */
int khq_layer_dense(const khq_layer* layer, void** k, void** vt, int* ld_vt, int* n_decoded);
/* Post-norm, pre-RoPE K [H_kv][256] of the token about to be stepped into
 * ring_u[write_pos % 256] (ref runtime.mojo:432-451). */
int khq_layer_capture_unroped(khq_layer* layer, const void* k_unroped, hipStream_t stream);
/* One decode step (ref runtime.mojo:454-613): ring write (k_unroped may be
 * NULL when captured before), compression event at the watermark, then the
 * two-region attention into out f16 [H_q][256].  Returns 1 when out was
 * written, 0 when neither region exists, -100 on bad arguments, -102 when the
 * raw window would exceed the ring (capacity reached), else an error code. */
int khq_layer_step(khq_layer* layer, const void* q_gate, const void* k_roped, const void* v,
                   const void* k_unroped, void* out, float scale, hipStream_t stream);
/* Chunked prefill of n tokens (no reference counterpart: the reference
 * prefills through n calls of khq_step, ref runtime.mojo:454-613, and this
 * reproduces those steps' results).  q_gate f16 [n][H_q][512], k_roped / v /
 * k_unroped f16 [n][H_kv][256], out f16 [n][H_q][256].  Token i is appended,
 * any compression event fires, and query i attends to the compressed prefix
 * and its raw window, as in step i; queries between events share one launch
 * (dense fp16 keys decoded from the compressed rows, MFMA attention).
 * Returns n, -100 on bad arguments, -102 at capacity, else an error code. */
int khq_layer_prefill(khq_layer* layer, const void* q_gate, const void* k_roped, const void* v,
                      const void* k_unroped, void* out, int n, float scale, hipStream_t stream);

/* ---- calibration dumps (replaces ref:src/models/qwen3_5/khq_dump.mojo) ----
 * A recorder of the two files the calibration reads:
 *   <dir>/kv_dump.bin  ('KHQD'): u32 magic | u32 n_layers | u32 dim, then
 *       n_layers x (u32 layer_id | u32 n_tokens), then per layer n_tokens x dim
 *       f32 K rows followed by n_tokens x dim f32 V rows (khq_dump.mojo:9-14,
 *       319-368);
 *   <dir>/attn_<layer>.bin ('KHQA'): u32 magic | u32 H_q | u32 H_kv | u32 D,
 *       then per token u32 n_valid (= pos + 1) and H_q x n_valid fp16 softmax
 *       scores (khq_dump.mojo:87-93, 199-316).
 * flags: KHQ_DUMP_KV and/or KHQ_DUMP_ATTN.  Returns NULL on bad arguments. */
#define KHQ_DUMP_KV 1
#define KHQ_DUMP_ATTN 2
typedef struct khq_dump khq_dump;
/* Replaces khq_dump_configure (khq_dump.mojo:28-39); kv_dim = H_kv * head_dim. */
khq_dump* khq_dump_create(const char* dir, int max_tokens, int kv_dim, int flags);
void khq_dump_destroy(khq_dump* dump);
/* Tokens recorded so far for `layer` (KHQD). */
int khq_dump_count(const khq_dump* dump, int layer);
/* Replaces khq_dump_kv (khq_dump.mojo:46-85): appends one token's post-norm,
 * pre-RoPE K and its V (f16 [kv_dim] each, device) to layer `layer`'s rows, as
 * an asynchronous device copy on `stream`; ignored once max_tokens are held. */
int khq_dump_kv(khq_dump* dump, int layer, const void* k, const void* v, hipStream_t stream);
/* Replaces khq_dump_attn (khq_dump.mojo:199-316): appends this token's roped K
 * (f16 [H_kv][D]) to the layer's history row `pos` (pos 0 clears it), computes
 * on the GPU the softmax over rows 0..pos of scale * q.k for every query head
 * (q = first D halves of each q_gate row [H_q][2 D]) and writes the record to
 * attn_<layer>.bin; synchronises `stream`.  Ignored for pos >= max_tokens or a
 * shape that differs from the first call's; -104 on a file error. */
int khq_dump_attn(khq_dump* dump, int layer, const void* q_gate, const void* k_roped, int pos,
                  int H_q, int H_kv, int D, float scale, hipStream_t stream);
/* Replaces khq_dump_flush (khq_dump.mojo:319-368): closes the KHQA files and
 * writes kv_dump.bin (no file when nothing was recorded), then restarts the
 * KHQD recording.  Synchronises the device. */
int khq_dump_flush(khq_dump* dump);

/* ---- calibration (replaces the calibration entry points of
 * ref:src/csrc/qmv_sm75_kernel.cu:4434-4810, driven by
 * ref:src/khq/calib.mojo:285-566; host driver: khq/calib.py) ----
 * All pointers are f32 device buffers; rows = i1.  Synchronous for ops
 * 2 and 4..9.  Returns 0, -100 on bad arguments, -1 for an unknown op, else a
 * hipError_t.  Ops (argument roles as in the reference):
 *   1 FWHT base     a x[rows][256], b d[256] -> e norms[rows],
 *                   f base = FWHT(x fp16(d) / norm) / 16
 *   2 K static      a proj -> f cents[4][256] = [0, -c, c, c], g ts
 *                   (c = 0.935 sigma ts, ts = 16 / sqrt(sum 0.528756 c0^2 + 0.464545 sigma^2))
 *   3 rotate        a rows, b rotor[64][16] -> e rows R^T per patch
 *   4 PCA           a FWHT-domain rows -> e rotor (columns: eigenvectors 2, 3, 4, 1
 *                   by decreasing eigenvalue)
 *   5 k-means 4     a rows -> e cents[4][256] (20 Lloyd iterations per dim)
 *   6 k-means VQ    a rotated rows -> e codebook[64][256][3] (30 iterations, seed i2)
 *   7 Procrustes    a rows, b codebook, e rotor in/out (i2 Lloyd iterations)
 *   8 SmartK        a x32, b x16, c d_k, d rotor, e cents, f1 ts -> f cents, g (ts, alpha)
 *   9 SmartV        a x32, b x16, c d_v, d rotor, e cents, f codebook, f1 ts -> g (ts, alpha)
 *  10 head-major    a rows [i1 tokens][i2 heads][256] -> e [i2][i1][256] */
int launch_cal_op(int op, const void* a, const void* b, const void* c, const void* d, void* e,
                  void* f, void* g, float f1, float f2, int i1, int i2, int i3, int i4,
                  hipStream_t stream);

/* SmartVQ tournament (replaces launch_cal_svq_train, ref .cu:4434-4596):
 * v f32 [N][256] head-major FWHT-domain V rows (N = H_kv * T), attn f32
 * [H_q][T][T] softmax scores (NULL: plain reconstruction loss), init_cb and
 * out_cb f32 [64][256][3], rp f32 [64][16]; out_wtrm f32 [256][256] = I + A B
 * of the winner (may be NULL).  Seeds 42, 137, 271 (n_seeds <= 3): 30 steps
 * each, then the remaining iterations for each, best attention-MSE proxy
 * first; the winner has the smallest proxy.  Synchronous. */
int launch_cal_svq_train(const void* v, const void* attn, const void* init_cb, const void* rp,
                         void* out_cb, void* out_wtrm, int N, int T, int H_q, int H_kv,
                         int iterations, int n_seeds, float lr, hipStream_t stream);

/* One SmartVQ pass (no counterpart in the reference: it exposes, for tests,
 * the step that launch_cal_svq_train repeats, ref .cu:2470-2530): forward and
 * gradients at codebook cb f32 [64][256][3] and transform factors wa f32
 * [256][8], wb f32 [8][256], temperature temp.  out_grad f32 [49152 + 2048 +
 * 2048] = d/d cb, d/d wa, d/d wb (the straight-through codebook gradient;
 * zero transform gradients without attn); out_loss f32 [2] = reconstruction
 * and dict losses.  Other arguments as launch_cal_svq_train.  Synchronous. */
int launch_cal_svq_pass(const void* v, const void* attn, const void* cb, const void* wa,
                        const void* wb, const void* rp, void* out_grad, void* out_loss, int N,
                        int T, int H_q, int H_kv, float temp, hipStream_t stream);

/* Attaches a dump recorder to a layer (NULL detaches): its
 * khq_layer_attention_step then records the token under `layer_id`
 * (ref attention.mojo:340-341, 355-356).  The recorder is not owned. */
int khq_layer_set_dump(khq_layer* layer, khq_dump* dump, int layer_id);

/* Replaces the KHQ part of qwen3_5_gated_attention_step_gpu_from_proj
 * (ref:src/models/qwen3_5/attention.mojo:319-365) for one token, from the
 * projections: head RMSNorm of q (q_gate [H_q][512], the q halves, in place)
 * and of k ([H_kv][256], in place) with optional f32 [256] weights (NULL = no
 * weight, the has_norms = False path) and eps; the normed pre-RoPE K captured
 * into ring_u; half-split RoPE of dims 0..63 at position `pos` (base = the
 * layer's rope_base) on q and k; the roped K and v written to the ring; the
 * attached dumps, if any; then khq_step (compression event, two-region
 * attention, merge, gate) into out f16 [H_q][256].  q_gate and k hold the
 * normed, roped values afterwards, as in the reference.  Returns as
 * khq_layer_step. */
int khq_layer_attention_step(khq_layer* layer, void* q_gate, void* k, const void* v,
                             const float* q_norm_w, const float* k_norm_w, float eps, int pos,
                             void* out, float scale, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KHQ_H */
