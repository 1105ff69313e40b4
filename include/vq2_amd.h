/*
 * vq2_amd.h -- C ABI of the MI355X-native VQ2 decode hot path
 * (libvq2_amd.so, HIP kernels for gfx950).
 *
 * Conventions
 *   - Every entry returns an int status: VQ2_OK (0) or a VQ2_ERR_* code.  On
 *     error, vq2_last_error() returns a thread-local message.  No entry aborts.
 *   - All pointers are device pointers unless stated otherwise; every array is
 *     dense (C-contiguous) with the strides given in elements.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Entries only
 *     enqueue work: no allocation, no host synchronisation, so they can be
 *     captured in a HIP graph.
 *   - Index planes hold uint16 codes stored as int16 bit patterns and are
 *     decoded as (int32)v & 0xFFFF; uint8 stage-2 planes are used as is.
 *   - Activations, codebooks, scales and outputs take a dtype code
 *     (VQ2_DT_*); all arithmetic is fp32.
 *
 * Reference interfaces (paths relative to the reference repository) are
 * cited beside each entry.
 */
#ifndef VQ2_AMD_H
#define VQ2_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element dtypes */
#define VQ2_DT_F32 0
#define VQ2_DT_F16 1
#define VQ2_DT_BF16 2

/* stage-2 index plane kinds */
#define VQ2_S2_NONE 0 /* cfg (16,):   2 bpw, one int16 plane                        */
#define VQ2_S2_U8 1   /* cfg (16,8):  3 bpw, + uint8 plane into a 256 x 8 codebook   */
#define VQ2_S2_U16 2  /* cfg (16,16): 4 bpw, + int16 plane into a 65536 x 8 codebook */

/* expert-id dtypes */
#define VQ2_ID_I32 0
#define VQ2_ID_I64 1

/* status codes */
#define VQ2_OK 0
#define VQ2_ERR_ARG 1         /* null pointer, bad size, dtype or alignment */
#define VQ2_ERR_HIP 2         /* a HIP runtime call failed                  */
#define VQ2_ERR_UNSUPPORTED 3 /* valid but unsupported shape               */

/* Library version (major*10000 + minor*100 + patch). */
int vq2_version(void);

/* Thread-local description of the last error on this thread ("" if none). */
const char* vq2_last_error(void);

/* Dense VQ GEMV, batched:  y[b, r] = (sum_k W[r, k] * x[b, k]) * scale[r] * rs
 * with W[r, 8g+j] = cb0[i0[r,g]][j] (+ cb1[i1[r,g]][j] for 3/4 bpw).
 *   x      [batch, x_stride] (n used), dtype x_dt
 *   idx0   [out_rows, n/8] int16;  idx1 [out_rows, n/8] uint8 (S2_U8) or int16 (S2_U16) or NULL
 *   cb0    [65536, 8];  cb1 [256, 8] (S2_U8) or [65536, 8] (S2_U16), both dtype cb_dt, 16-byte aligned
 *   scale  [out_rows] dtype s_dt;   y [batch, y_stride] dtype y_dt
 * n must be a multiple of 8.
 * Replaces vq_gemv_16 (vq2/kernels.py:224-230) and vq_gemv_16_8
 * (vq2/kernels.py:215-221); adds the (16,16) 4 bpw variant (the reference's
 * PackedLinear.weight_rows + F.linear fallback, vq2/runtime.py:82-110) and
 * batch > 1 (same fallback). */
int vq2_gemv(const void* x, int x_dt, int64_t batch, int64_t x_stride,
             const int16_t* idx0, const void* idx1, int s2_kind,
             const void* cb0, const void* cb1, int cb_dt,
             const void* scale, int s_dt,
             void* y, int y_dt, int64_t y_stride,
             int64_t out_rows, int64_t n, float rs, void* stream);

/* Small-M batched VQ GEMM on the matrix cores (v_mfma_f32_16x16x32_f16):
 * y[b * y_stride + r] = (sum_k x[b * x_stride + k] * W[r, k]) * s[r] * rs for
 * b < batch (1..64), x already rotated, n % 64 == 0, 16-byte aligned index
 * planes and activation rows.  Every centroid is gathered once for all batch
 * rows (vq2_gemv gathers it once per 8-row batch tile).  The activation is
 * rounded to fp16 under a power-of-two scale per row and K split (and bf16 /
 * fp32 centroids to fp16); accumulation is fp32.  K is split across
 * workgroups to fill the device; the raw partials then go to `workspace`
 * (vq2_gemm_small_m_workspace(...) bytes, 16-byte aligned, 0 = none needed;
 * contents on entry do not matter) and a second launch sums them in a fixed
 * order.  Replaces the PackedLinear batch > 1 fallback, dequantize + F.linear
 * (vq2/runtime.py:82-89, 105-110). */
size_t vq2_gemm_small_m_workspace(int64_t batch, int64_t out_rows, int64_t n);
int vq2_gemm_small_m(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                     const int16_t* idx0, const void* idx1, int s2_kind,
                     const void* cb0, const void* cb1, int cb_dt,
                     const void* scale, int s_dt,
                     void* y, int y_dt, int64_t y_stride,
                     int64_t out_rows, int64_t n, float rs,
                     void* workspace, size_t ws_bytes, void* stream);

/* vq2_gemm_small_m without the workspace arguments: allocates nothing.  No
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops and harnesses that
 * forbid hipMalloc).  The split-K partials go to a device array of the
 * library instead, VQ2_NOALLOC_SCRATCH_BYTES (16 MiB) per GPU, held until the
 * process ends; a shape whose partials need more (vq2_gemm_small_m_workspace
 * (batch, out_rows, n) > VQ2_NOALLOC_SCRATCH_BYTES, e.g. a 151936-row LM head
 * at batch 64) returns VQ2_ERR_UNSUPPORTED without launching.  Every call on
 * one GPU shares that array and leaves its partials there: calls that overlap
 * on one GPU (several streams or host threads) race, so serialise them.  The
 * stream's device must be the current device.  Results equal
 * vq2_gemm_small_m's bit for bit (same kernels and plan). */
#define VQ2_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int vq2_gemm_small_m_noalloc(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                             const int16_t* idx0, const void* idx1, int s2_kind,
                             const void* cb0, const void* cb1, int cb_dt,
                             const void* scale, int s_dt,
                             void* y, int y_dt, int64_t y_stride,
                             int64_t out_rows, int64_t n, float rs, void* stream);

/* vq2_gemm_small_m followed by the top-1 of every activation row, without
 * writing the logits: out_idx[b] = argmax_r y[b, r] (torch.argmax's first
 * maximum; int64, 8-byte aligned), out_val[b] = y[b, out_idx[b]] (fp32, may
 * be NULL), with y computed exactly as vq2_gemm_small_m computes it in fp32.
 * The partials sum and the scale go into one reduce launch that keeps each
 * block's best key, and a last launch picks the winner.  `workspace`:
 * vq2_gemm_small_m_argmax_workspace(...) bytes, 16-byte aligned, contents on
 * entry do not matter.  Replaces PackedLMHead.forward at batch > 1
 * (vq2/runtime.py:136-144, 105-110) + torch.argmax (legion/engine.py:288). */
size_t vq2_gemm_small_m_argmax_workspace(int64_t batch, int64_t out_rows, int64_t n);
int vq2_gemm_small_m_argmax(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                            const int16_t* idx0, const void* idx1, int s2_kind,
                            const void* cb0, const void* cb1, int cb_dt,
                            const void* scale, int s_dt,
                            int64_t out_rows, int64_t n, float rs,
                            void* workspace, size_t ws_bytes,
                            int64_t* out_idx, float* out_val, void* stream);

/* One matrix of a vq2_gemv_rht launch: index planes, row scales and output
 * (y [batch, y_stride], dtype of the launch), all device pointers. */
typedef struct vq2_seg {
    const int16_t* idx0; /* [out_rows, n/8] int16                                   */
    const void* idx1;    /* stage-2 plane or NULL (must match the launch's s2_kind) */
    const void* scale;   /* [out_rows]                                              */
    void* y;             /* [batch, y_stride]                                       */
    int64_t out_rows;
    int64_t y_stride;
} vq2_seg;

/* Rotate-then-multiply in one launch, for up to 4 matrices that read the same
 * activation (q/k/v, gate/up):
 *   xr[b] = RHT_fwd(x[b]) with perm/sign (nullable), hb-point blocks, scale
 *   segs[s].y[b, r] = (sum_k W_s[r, k] * xr[b, k]) * segs[s].scale[r] * rs
 * Every workgroup builds xr in LDS itself, so no rotated copy of x is written.
 * hb == 0: x is already rotated (perm, sign and rht_scale are ignored) --
 * for n > 2048 a separate vq2_rht launch is cheaper than rotating n values
 * in every workgroup.  Requires n % 64 == 0, 16-byte aligned index planes
 * and batch <= 2 (larger batches: vq2_rht + vq2_gemv); segs is a host array.
 * Replaces FastRot + vq_gemv_16 / vq_gemv_16_8 of PackedLinear.forward
 * (vq2/runtime.py:91-104) and Rot.fwd + F.linear of its fallback
 * (vq2/runtime.py:105-110). */
int vq2_gemv_rht(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                 const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                 int n_seg, const vq2_seg* segs,
                 int s2_kind, const void* cb0, const void* cb1, int cb_dt, int s_dt, int y_dt,
                 int64_t n, float rs, void* stream);


/* Grouped per-expert 2 bpw VQ GEMV over a device-resident expert pool:
 *   e = ids[k];  y[k, r] = (sum_g cb[pool[e, r, g]] . x_k[8g:8g+8]) * pool_scale[e, r] * rs
 *   x_k = x + (k / pairs_per_x) * x_pair_stride
 *         (stride 0: one activation shared by all pairs, as gate_up;
 *          stride n, pairs_per_x 1: one per pair, as down;
 *          stride n, pairs_per_x P: token t's activation for its P experts)
 *   ids    [n_pairs] int32/int64 on device (expert ids or slot ids); an id
 *          outside [0, n_experts) produces NaN rows instead of a fault
 *   pool   [n_experts, out_rows, ng] int16;  pool_scale [n_experts, out_rows]
 *   y      [n_pairs, y_pair_stride]
 * Replaces vq_moe_parallel_gate_up (vq2/kernels.py:246-254) and
 * vq_moe_parallel_down (vq2/kernels.py:256-264). */
int vq2_moe_grouped(const void* x, int x_dt, int64_t x_pair_stride, int64_t pairs_per_x,
                    const void* ids, int ids_dt, int64_t n_pairs,
                    const int16_t* pool, int64_t n_experts,
                    const void* cb, int cb_dt,
                    const void* pool_scale, int s_dt,
                    void* y, int y_dt, int64_t y_pair_stride,
                    int64_t out_rows, int64_t ng, float rs, void* stream);

/* Grouped gate_up with the activation rotation fused in: for token t and its
 * P experts ids[t*P + j],
 *   xr_t = RHT_fwd(h[t]) (perm/sign nullable, hb-point blocks, rht_scale)
 *   y[t*P + j, r] = (sum cb[pool[e, r, g]] . xr_t[8g:8g+8]) * pool_scale[e, r] * rs
 * h is [tokens, n] (n = ng * 8).  Replaces rot_2048.fwd + vq_moe_parallel_gate_up
 * of PagedMoEExpert.forward (vq2/paged_runtime.py:495-500). */
int vq2_moe_gate_up_rht(const void* h, int h_dt, int64_t tokens,
                        const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                        const void* ids, int ids_dt, int64_t P,
                        const int16_t* pool, int64_t n_experts,
                        const void* cb, int cb_dt, const void* pool_scale, int s_dt,
                        void* y, int y_dt, int64_t y_pair_stride,
                        int64_t out_rows, int64_t ng, float rs, void* stream);

/* vq2_moe_gate_up_rht with the router built in: every workgroup selects its
 * pair's expert from the token's router logits (softmax over n_routed, top-k,
 * renormalised; ties to the lower id, as vq2_router_topk) before it fetches
 * codes, so the MoE layer needs no separate router launch.  Pair p of token t
 * (P = k + 1 with a shared expert, else k) is slot p of the top-k, slot k the
 * shared expert shared_id (-1: none) weighted sigmoid(shared_gate . h_t).
 * Outputs the same ids / w (int32 / fp32 [tokens, P]) as vq2_router_topk,
 * for vq2_moe_down_swiglu_combine.  Replaces Qwen3_5MoeTopKRouter.forward
 * (HF:760-776) + rot_2048.fwd + vq_moe_parallel_gate_up
 * (vq2/paged_runtime.py:495-500, vq2/kernels.py:246-254). */
int vq2_moe_router_gate_up_rht(const void* h, int h_dt, int64_t tokens,
                               const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                               const void* logits, int l_dt, int64_t n_routed, int k,
                               const void* shared_gate, int g_dt, int64_t shared_id,
                               const int16_t* pool, int64_t n_experts,
                               const void* cb, int cb_dt, const void* pool_scale, int s_dt,
                               void* y, int y_dt, int64_t y_pair_stride,
                               int64_t out_rows, int64_t ng, float rs,
                               int32_t* ids, float* w, void* stream);

/* Grouped down projection fused with the weighted expert combine:
 *   out[t, r] = sum_{j < P} w[t*P+j] * (VQ(pool[ids[t*P+j]]) x_{t*P+j})[r]
 * with x_p = x + p * ng*8 and each term (acc * scale) * rs as in
 * vq2_moe_grouped.  w is fp32 [tokens*P] on device.
 * Replaces the vq_moe_parallel_down call plus (y_down * topk_w[:, None]).sum(0)
 * of PagedMoEExpert.forward (vq2/paged_runtime.py:505-510). */
int vq2_moe_down_combine(const void* x, int x_dt,
                         const void* ids, int ids_dt, const float* w, int64_t tokens, int64_t P,
                         const int16_t* pool, int64_t n_experts,
                         const void* cb, int cb_dt,
                         const void* pool_scale, int s_dt,
                         void* out, int out_dt, int64_t out_stride,
                         int64_t out_rows, int64_t ng, float rs, void* stream);

/* The whole expert epilogue in one launch: for token t and pair p = t*P + j,
 *   act_p = RHT_fwd(silu(gu[p, :n]) * gu[p, n:2n])   (n = ng * 8, in LDS)
 *   out[t, r] = sum_j w[p] * (sum_k VQ(pool[ids[p]])[r, k] * act_p[k]) * scale * rs
 * Replaces the SwiGLU, rot_512.fwd, vq_moe_parallel_down and the weighted sum
 * of PagedMoEExpert.forward (vq2/paged_runtime.py:501-510). */
int vq2_moe_down_swiglu_combine(const void* gu, int gu_dt, int64_t gu_stride,
                                const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                                const void* ids, int ids_dt, const float* w, int64_t tokens, int64_t P,
                                const int16_t* pool, int64_t n_experts,
                                const void* cb, int cb_dt, const void* pool_scale, int s_dt,
                                void* out, int out_dt, int64_t out_stride,
                                int64_t out_rows, int64_t ng, float rs, void* stream);

/* Promoted 3 bpw experts: vq2_moe_gate_up_rht and vq2_moe_down_swiglu_combine
 * over (16,8) pools -- pool int16 [E, rows, ng] stage-1 codes, pool1 uint8
 * [E, rows, ng] stage-2 codes, cb [65536, 8], cb1 [256, 8] (same dtype):
 *   W[e, r, 8g:8g+8] = (cb[pool[e, r, g]] + cb1[pool1[e, r, g]]) * pool_scale[e, r]
 * accumulate != 0 makes the combine add into out (out += sum_j ...), so the
 * 2 bpw and the 3 bpw experts of one token sum into one output.
 * Replace the dense path of promoted experts in PagedMoEExpert: stage-1 +
 * stage-2 dequant, rot.inv and F.linear per expert (vq2/paged_runtime.py:
 * 357-389 at load, 446-458 and 514-521 per token). */
int vq2_moe_gate_up_rht_16_8(const void* h, int h_dt, int64_t tokens,
                             const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                             const void* ids, int ids_dt, int64_t P,
                             const int16_t* pool, const uint8_t* pool1, int64_t n_experts,
                             const void* cb, const void* cb1, int cb_dt, const void* pool_scale, int s_dt,
                             void* y, int y_dt, int64_t y_pair_stride,
                             int64_t out_rows, int64_t ng, float rs, void* stream);
int vq2_moe_down_swiglu_combine_16_8(const void* gu, int gu_dt, int64_t gu_stride,
                                     const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                                     const void* ids, int ids_dt, const float* w, int64_t tokens, int64_t P,
                                     const int16_t* pool, const uint8_t* pool1, int64_t n_experts,
                                     const void* cb, const void* cb1, int cb_dt, const void* pool_scale, int s_dt,
                                     void* out, int out_dt, int64_t out_stride,
                                     int64_t out_rows, int64_t ng, float rs, int accumulate, void* stream);

/* Randomised Hadamard transform over the last dim, hb-point blocks:
 *   forward: v[i] = x[perm[i]] * sign[i];  y_blk = H_hb v_blk * scale
 *   inverse: z_blk = H_hb x_blk * scale;   y[perm[i]] = z[i] * sign[i]
 * H_hb is the Sylvester Hadamard matrix (natural order).  perm (int32 [n])
 * and sign (int8 +-1 [n]) may be NULL (identity / all +1).  hb is a power of
 * two in [2, 8192] dividing n.  x and y must not overlap.
 * Replaces Rot.fwd / Rot.inv (vq2/vq.py:74-87) and FastRot.__call__
 * (vq2/runtime.py:57-63, which is scale = 1). */
int vq2_rht(const void* x, int x_dt, int64_t x_stride,
            void* y, int y_dt, int64_t y_stride,
            const int32_t* perm, const int8_t* sign,
            int64_t n, int64_t hb, int64_t batch, float scale, int inverse, void* stream);

/* MoE expert epilogue fused with the intermediate RHT:
 *   act = silu(gu[b, :inter]) * gu[b, inter:2*inter];  y[b] = RHT_fwd(act)
 * Replaces act = (silu(gate.f32) * up.f32) and rot_512.fwd(act) of
 * PagedMoEExpert.forward (vq2/paged_runtime.py:501-504). */
int vq2_swiglu_rht(const void* gu, int gu_dt, int64_t gu_stride, int64_t inter,
                   void* y, int y_dt, int64_t y_stride,
                   const int32_t* perm, const int8_t* sign,
                   int64_t hb, int64_t batch, float scale, void* stream);

/* Top-k router on given logits, per token (transformers 5.15.0
 * Qwen3_5MoeTopKRouter.forward: softmax in fp32 -> topk -> renormalise):
 *   ids[t, j] (int32), w[t, j] (fp32), j < k, in descending-probability order
 *   (ties toward the lower expert id).  Row stride of ids/w is k + extra.
 * If shared_id >= 0, slot k of each row gets the shared expert:
 *   ids[t, k] = shared_id,  w[t, k] = sigmoid(sum_i gate[i] * h[t, i])
 * (Qwen3_5MoeSparseMoeBlock.forward shared-expert gate), with h [tokens, hidden].
 * n_experts <= 1024, k <= 32. */
int vq2_router_topk(const void* logits, int l_dt, int64_t tokens, int64_t n_experts, int k,
                    const void* h, int h_dt, int64_t hidden, const void* gate, int g_dt, int64_t shared_id,
                    int32_t* ids, float* w, void* stream);

/* First-maximum index per row (torch.argmax semantics for NaN-free rows):
 *   out_idx[r] = argmax_c v[r, c]   (int64), out_val[r] = v[r, out_idx[r]] (fp32, may be NULL)
 * Replaces torch.argmax over logits (legion/engine.py:288, vq2/generate.py:65). */
int vq2_argmax_rows(const void* v, int v_dt, int64_t rows, int64_t cols,
                    int64_t* out_idx, float* out_val, void* stream);

/* LM head + top-1 of each batch column (torch.argmax's first maximum).
 * batch 1, n % 8 == 0, n <= 2048 (one K chunk per wave), out_rows >= 8: fused
 * -- the GEMV keeps each workgroup's best (value, row) and one small launch
 * picks the winner, no logits are written (`logits_ws` holds the per-
 * workgroup keys).  Otherwise the logits go to `logits_ws` [batch, out_rows]
 * (fp32) and vq2_argmax_rows follows.  logits_ws and out_idx 8-byte aligned.
 * Replaces PackedLMHead.forward (vq2/runtime.py:136-144) + torch.argmax. */
int vq2_gemv_argmax(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                    const int16_t* idx0, const void* idx1, int s2_kind,
                    const void* cb0, const void* cb1, int cb_dt,
                    const void* scale, int s_dt,
                    int64_t out_rows, int64_t n, float rs,
                    float* logits_ws, int64_t* out_idx, float* out_val, void* stream);

/* Code-sorted internal layout of one VQ matrix (2 or 4 bpw), for the batch-1
 * GEMV of large matrices.  The reference's int16 index planes stay the
 * public format; this repack is built once at load time, on the host, and
 * lets the lanes of a wave share codebook lines: random 16-byte centroid
 * gathers are capped by the L2 request rate, sorted ones are not.
 *   rows are cut into n_chunks = ceil(out_rows / rows_per_chunk) chunks
 *   (rows_per_chunk at most min(2^(17 - ceil(log2 ng)) - 1, 511);
 *   vq2_sorted_rows_per_chunk gives the default: at most
 *   min(2^(16 - ceil(log2 ng)) - 1, 255) rows, over a multiple of
 *   chunk_align chunks when the chunks keep >= 128 rows, e.g. chunk_align =
 *   the CU count; with chunk_align > 1 a matrix of fewer than 2^20 codes
 *   takes ceil(4 out_rows / (3 chunk_align)) rows per chunk (about 0.75 x
 *   chunk_align chunks), at most 64; a matrix tall enough that a multiple of 2 x chunk_align
 *   chunks of more rows (up to the first limit) covers it takes those, e.g.
 *   a 151,936-row LM head: 512 chunks of 297 rows) of near-equal height:
 *   chunk c holds rows
 *   [c * rb + min(c, nbig), + rb + (c < nbig)), rb = out_rows / n_chunks,
 *   nbig = out_rows % n_chunks; a chunk's codes are sorted by value and
 *   dealt into 64-lane instructions in which no row repeats within a
 *   32-lane half (lanes 0-31, 32-62), or within a 16-lane quarter (lanes
 *   0-15, 16-31, 32-47, 48-62) for chunks of at most 32 rows (expert pools,
 *   vq2_sorted_pack_pool: halves at any height); lane 63 carries the instruction's
 *   base code (its smallest), every other lane one code as the 24-bit field
 *   (code - base) << P | row_in_chunk << ceil(log2 ng) | group, P =
 *   ceil(log2 ng) + bitlen(rows_per_chunk) <= 17 (an instruction is closed
 *   before an offset would reach 2^(24 - P)); 4 instructions form an
 *   iteration of 192 uint32 (768 bytes): lane l's three words at 3 l are
 *   lo16(F0) | lo16(F1) << 16, lo16(F2) | lo16(F3) << 16 and the four
 *   fields' high bytes (lane 63: the four base codes, then 0); every
 *   chunk's stage-1 and stage-2 entries are padded (dummy row, offset 0) to
 *   the matrix's largest stage-1 / stage-2 iteration counts, so chunk c
 *   holds iterations [c * ipc, (c + 1) * ipc), its stage-2 ones from
 *   c * ipc + stage1_iters on.  3 bytes per code.
 * vq2_sorted_pack (host memory, no GPU work) fills `entries` (up to
 * cap_iters * 192 uint32, 16-byte aligned) and sets *iters_per_chunk
 * (ipc), *stage1_iters and *n_iters = n_chunks * ipc, n_chunks =
 * ceil(out_rows / rows_per_chunk) (also when the capacity is too small,
 * which returns VQ2_ERR_ARG).  idx1 (the stage-2 plane as int16: (16,16), or
 * a (16,8) uint8 plane widened to int16 values 0..255) may be NULL; n_threads
 * <= 0: all host threads.  No reference counterpart (a load-time transform
 * of the planes PackedLinear holds, vq2/runtime.py:70-80). */
int64_t vq2_sorted_rows_per_chunk(int64_t out_rows, int64_t ng, int64_t chunk_align);
int vq2_sorted_pack(const int16_t* idx0, const int16_t* idx1, int64_t out_rows, int64_t ng, int64_t rows_per_chunk,
                    uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk, int64_t* stage1_iters,
                    int64_t* n_iters, int n_threads);

/* The workspace of vq2_sorted_gemv begins with VQ2_SORTED_WS_HEADER bytes
 * of arrival counters: the slices of a chunk are summed inside the launch
 * by the chunk's workgroup that arrives last.  The header must be zero
 * before the first call that uses the workspace (e.g. allocate it zeroed);
 * every call leaves it zero.  One workspace may serve all vq2_sorted_gemv
 * calls of a stream; calls that share a workspace must not run
 * concurrently.  A launch with several slices has at most
 * VQ2_SORTED_MAX_COUNTERS chunks. */
#define VQ2_SORTED_WS_HEADER 16384
/* The header's last 128-byte line holds vq2_sorted_moe's status word
 * (below); counters use the words before it. */
#define VQ2_SORTED_WS_STATUS (VQ2_SORTED_WS_HEADER - 128)
#define VQ2_SORTED_MAX_COUNTERS (VQ2_SORTED_WS_STATUS / 4)

/* One packed matrix of a sorted launch (device pointers, except the struct). */
typedef struct vq2_sorted_mat {
    const uint32_t* entries;  /* from vq2_sorted_pack, copied to the device    */
    int64_t iters_per_chunk;  /* the values vq2_sorted_pack set                */
    int64_t stage1_iters;
    int64_t n_iters;
    int64_t rows_per_chunk;   /* the value the matrix was packed with          */
    int has_stage2;           /* 0: none; 1: packed with an int16 idx1 ((16,16),
                                 cb1 [65536, 8]); 2: packed with a uint8 idx1
                                 widened to int16 ((16,8), cb1 [256, 8], codes
                                 masked to 8 bits)                             */
    const void* scale;        /* [out_rows], dtype s_dt                        */
    void* y;                  /* [out_rows], dtype y_dt (unused by the top-1) */
    int64_t out_rows;
} vq2_sorted_mat;

/* Batch-1 VQ GEMV of up to 4 packed matrices sharing the activation, with
 * the RHT of x built in the kernel's LDS (hb > 0: perm / sign nullable,
 * rht_scale; n % 64 == 0, x 16-byte aligned) or x already rotated (hb == 0):
 *   y_m[r] = (sum_k W_m[r, k] * xr[k]) * scale_m[r] * rs
 * fp16 / bf16 codebooks.  `slices` workgroups share each chunk; with more
 * than one the raw partials go to `workspace` (vq2_sorted_gemv_workspace
 * bytes, zeroed header) and the chunk's last workgroup to finish sums them
 * in slice order (one launch; deterministic).  Replaces FastRot +
 * vq_gemv_16 of PackedLinear.forward (vq2/runtime.py:91-104) and its
 * (16,16) fallback (vq2/runtime.py:105-110) for large matrices. */
size_t vq2_sorted_gemv_workspace(const vq2_sorted_mat* mats, int n_mat, int slices);
int vq2_sorted_gemv(const void* x, int x_dt, const int32_t* perm, const int8_t* sign, int64_t hb, float rht_scale,
                    int n_mat, const vq2_sorted_mat* mats, const void* cb0, const void* cb1, int cb_dt, int s_dt,
                    int y_dt, int64_t n, float rs, int slices, void* workspace, size_t ws_bytes, void* stream);

/* LM head + top-1 over one packed matrix at batch 1: out_idx[0] = argmax_r
 * y[r] (first maximum), out_val[0] = y[out_idx[0]] (may be NULL), with y as
 * vq2_sorted_gemv computes it; no logits are written.  `workspace`:
 * vq2_sorted_gemv_argmax_workspace bytes (one key per chunk).  Replaces
 * PackedLMHead.forward (vq2/runtime.py:136-144) + torch.argmax
 * (legion/engine.py:288). */
size_t vq2_sorted_gemv_argmax_workspace(const vq2_sorted_mat* mat);
int vq2_sorted_gemv_argmax(const void* x, int x_dt, const int32_t* perm, const int8_t* sign, int64_t hb,
                           float rht_scale, const vq2_sorted_mat* mat, const void* cb0, const void* cb1, int cb_dt,
                           int s_dt, int64_t n, float rs, void* workspace, size_t ws_bytes, int64_t* out_idx,
                           float* out_val, void* stream);

/* VQ GEMM of batch = 1..4 activation rows over up to 4 packed matrices:
 *   y_m[b * out_rows + r] = (sum_k W_m[r, k] * xr[b * x_stride + k]) * scale_m[r] * rs
 * with xr already rotated (16-byte aligned, x_stride >= n, a multiple of 8)
 * and every output y_m [batch, out_rows].  One centroid gather serves every
 * activation row.  The activation is held in fp16 with a power-of-two
 * scale per row (fp16 activations as they are; ~1e-4 of max |y|), all sums
 * in fp32.  `slices` workgroups share each chunk; with more than one,
 * `workspace` (vq2_sorted_gemm_batch_workspace bytes, header zero as for
 * vq2_sorted_gemv, which it may share) holds the partials and the chunk's
 * last workgroup sums them in slice order (deterministic).  A workgroup
 * holds 2 activation rows (batch <= 2) or 4 in
 * max(n * rows / 2, 512 * rows) * 4 + 32 * parts * (rows_per_chunk + 1) *
 * rows bytes of LDS (parts = 4 for chunks of at most 32 rows, else 2);
 * at batch 3-4 a call whose 4-row workgroups would exceed 80 KiB (one per
 * CU) runs 2-row workgroups instead: with one slice, one launch over both
 * row pairs and one final top-1 (the LM head's 297-row chunks: 18 % faster
 * at batch 4); with several, two launches sharing the workspace in stream
 * order.  More than
 * 150 KiB for the rows of a launch gives VQ2_ERR_UNSUPPORTED (n = 2048 fits
 * with any chunk height, n = 6144 with 62-row chunks, n = 32768 at 2 rows).
 * Replaces the PackedLinear batch > 1
 * fallback, dequant + F.linear (vq2/runtime.py:82-89, 105-110). */
size_t vq2_sorted_gemm_batch_workspace(const vq2_sorted_mat* mats, int n_mat, int64_t batch, int slices);
int vq2_sorted_gemm_batch(const void* x, int x_dt, int64_t batch, int64_t x_stride, int n_mat,
                          const vq2_sorted_mat* mats, const void* cb0, const void* cb1, int cb_dt, int s_dt, int y_dt,
                          int64_t n, float rs, int slices, void* workspace, size_t ws_bytes, void* stream);

/* vq2_sorted_gemm_batch of one matrix followed by the top-1 of every
 * activation row, without writing logits: out_idx[b] = argmax_r y[b, r]
 * (first maximum; int64, 8-byte aligned), out_val[b] = y[b, out_idx[b]]
 * (may be NULL).  `workspace`: vq2_sorted_gemm_batch_argmax_workspace bytes
 * (one key per chunk and row, 8-byte aligned).  Replaces PackedLMHead.forward
 * at batch > 1 (vq2/runtime.py:136-144, 105-110) + torch.argmax
 * (legion/engine.py:288). */
size_t vq2_sorted_gemm_batch_argmax_workspace(const vq2_sorted_mat* mat, int64_t batch);
int vq2_sorted_gemm_batch_argmax(const void* x, int x_dt, int64_t batch, int64_t x_stride,
                                 const vq2_sorted_mat* mat, const void* cb0, const void* cb1, int cb_dt, int s_dt,
                                 int64_t n, float rs, void* workspace, size_t ws_bytes, int64_t* out_idx,
                                 float* out_val, void* stream);

/* ---- MoE experts over code-sorted expert pools -------------------------
 * vq2_sorted_pack_pool (host memory, no GPU work) packs an expert pool
 * idx [n_experts, rows, ng] (the int16 stage-1 plane; idx1, the stage-2
 * plane as int16 -- a (16,8) uint8 plane widened to values 0..255 -- or
 * NULL) expert by expert, each as vq2_sorted_pack packs a matrix with the
 * same rows_per_chunk R (at most min(2^(16 - ceil(log2 ng)) - 1, 511): pools
 * keep 16-bit positions; and 32-lane halves at every R, where
 * vq2_sorted_pack takes quarters for R <= 32), and pads every chunk's stage-1 and stage-2 entries
 * (dummy-row entries) to the pool's largest counts, so chunk c of expert e
 * holds iterations [(e * C + c) * ipc, (e * C + c + 1) * ipc), C =
 * ceil(rows / R), its stage-2 ones from *stage1_iters on.  *n_iters =
 * n_experts * C * ipc; capacity as vq2_sorted_pack.  No reference
 * counterpart (a load-time transform of the pools PackedMoEExpertUniversal
 * holds, vq2/load_and_test_full_35b.py:31-47, and of the promoted 3 bpw
 * experts of vq2/paged_runtime.py:357-389). */
int vq2_sorted_pack_pool(const int16_t* idx, const int16_t* idx1, int64_t n_experts, int64_t rows, int64_t ng,
                         int64_t rows_per_chunk, uint32_t* entries, int64_t cap_iters, int64_t* iters_per_chunk,
                         int64_t* stage1_iters, int64_t* n_iters, int n_threads);

/* One packed expert pool (device pointers, except the struct). */
typedef struct vq2_sorted_pool {
    const uint32_t* entries;  /* from vq2_sorted_pack_pool                     */
    int64_t iters_per_chunk;
    int64_t n_iters;
    int64_t rows_per_chunk;
    int64_t rows;             /* rows per expert                               */
    int64_t ng;               /* groups per row (input width / 8)              */
    const void* scale;        /* [n_experts, rows], dtype scale_dt             */
    int scale_dt;
    int64_t stage1_iters;     /* = iters_per_chunk without a stage 2           */
    int has_stage2;           /* 0; 1: int16 stage 2, cb1 [65536, 8]; 2: the
                                 uint8 stage 2 of (16,8), cb1 [256, 8]         */
    const void* cb1;          /* stage-2 codebook in the dtype of cb, or NULL  */
} vq2_sorted_pool;

/* The permutation, signs, block size and scale of one rotation. */
typedef struct vq2_rot_tables {
    const int32_t* perm;      /* [n] or NULL (16-byte aligned)                 */
    const int8_t* sign;       /* [n] or NULL (8-byte aligned)                  */
    int64_t hb;
    float scale;
} vq2_rot_tables;

/* The experts of an MoE layer for `tokens` tokens of h [tokens, hidden]:
 *   gu  = VQ(gate_up[e]) . RHT_h(h_t)           (pool [n_experts, 2 inter, hidden / 8])
 *   act = RHT_i(silu(gu[:inter]) * gu[inter:])
 *   out[t] = sum_k w[t, k] * VQ(down[e]) . act   (pool [n_experts, hidden, inter / 8])
 * with e = ids[t, k] over pairs_per_token pairs, or, with router logits
 * [tokens, n_routed] (logits != NULL), the router built in: softmax, top_k
 * (ties to the lower id), renormalised; the last pair (pairs_per_token =
 * top_k + 1) is the shared expert shared_id with weight
 * sigmoid(shared_gate . h_t); the ids / weights go to ids_out / w_out.
 * At most three launches (gate_up, down, combine), fp32 arithmetic, an id outside
 * the pool gives NaN for its token.  slices_gu / slices_dn workgroups share
 * each chunk; workspace: vq2_sorted_moe_workspace bytes, whose first
 * VQ2_SORTED_WS_HEADER bytes (per-pair counters) are zero before the first
 * call; every call leaves the counters zero.  For hidden 2048 / inter 512
 * and at most 127 pairs (a 128-byte count each) the
 * gate_up and down launches are one launch whose down workgroups wait
 * (bounded) on the per-pair counts of finished gate_up workgroups; calls
 * that share a workspace must not overlap.  A wait that gives up (the
 * dispatcher did not start the gate_up workgroups ahead of the down ones
 * that wait for them, or the count was unreachable) turns its pair's
 * output NaN and ORs VQ2_MOE_WAIT_ID (the router's published id) or
 * VQ2_MOE_WAIT_COUNT (the pair's gate_up count) into the uint32 status
 * word at byte VQ2_SORTED_WS_STATUS of the workspace; no kernel clears it
 * (vq2_sorted_moe_status reads it, and may clear it, synchronously).  Replaces the
 * per-token expert loop of PackedMoEExpertUniversal.forward
 * (vq2/load_and_test_full_35b.py:53-95) / PagedMoEExpert.forward
 * (vq2/paged_runtime.py:495-510), with the router, the transformers
 * Qwen3_5MoeSparseMoeBlock routing (softmax, top-k, shared expert gate). */
size_t vq2_sorted_moe_workspace(int64_t tokens, int pairs_per_token, int64_t hidden, int64_t inter, int slices_gu,
                                int slices_dn);
#define VQ2_MOE_WAIT_ID 1
#define VQ2_MOE_WAIT_COUNT 2
/* The status word of a vq2_sorted_moe workspace (device pointer), read after
 * the work queued on `stream` so far has finished; clear != 0 sets it back
 * to 0.  Returns the bits (>= 0) or a negative VQ2_ERR_*.  No reference
 * counterpart (the reference's expert loop has no cross-workgroup wait). */
int vq2_sorted_moe_status(void* workspace, int clear, void* stream);
/* Process-wide bound of each wait of the one-launch MoE (max_polls polls of
 * >= 640 clocks; default 2^20) and an offset added to the gate_up count the
 * down workgroups wait for (default 0).  For tests of the give-up path: a
 * short bound with an unreachable count makes every wait give up while
 * every kernel still exits normally.  No reference counterpart. */
int vq2_sorted_moe_set_wait(int64_t max_polls, int32_t extra_arrivals);
int vq2_sorted_moe(const void* h, int h_dt, int64_t tokens, int pairs_per_token,
                   const void* ids, int ids_i64, const float* w,
                   const void* logits, int l_dt, int64_t n_routed, int top_k, int64_t shared_id,
                   const void* shared_gate, int g_dt, int32_t* ids_out, float* w_out,
                   int64_t n_experts, int64_t hidden, int64_t inter,
                   const vq2_sorted_pool* gate_up, const vq2_sorted_pool* down, const void* cb, int cb_dt,
                   const vq2_rot_tables* rot_h, const vq2_rot_tables* rot_i, void* out, int out_dt,
                   int slices_gu, int slices_dn, void* workspace, size_t ws_bytes, void* stream);

/* ---- Device-resident expert pager ---------------------------------------
 * The slot tables of a paged expert pool on the device: slot_of
 * [n_experts] (slot or -1), expert_of [capacity] (expert or -1), stamp
 * [capacity] (step clock of the last use, -1 when never used; initialise
 * all three to -1) and state int32 [5] (clock, copies of the last step,
 * hits, misses, error bits: 1 = an expert id outside [0, n_experts),
 * 2 = more distinct experts in a step than slots; initialise to 0).
 * vq2_pager_step (one workgroup) pages one step's routed ids [n_pairs]
 * (int32 / int64): resident experts keep their slots, missing ones (distinct,
 * in pair order) take the least recently used slots the step does not use;
 * it writes pair_slot [n_pairs] (-1 for a pair it cannot serve) and the
 * (expert, slot) copies [n_pairs][2].  vq2_pager_copy then copies those
 * experts' records from `mirror`, pinned host memory holding the layer's
 * container records [n_experts][record_bytes] back to back (segments:
 * gate_up index plane, its fp16 scales, down index plane, its fp16 scales,
 * seg_bytes[4], each a multiple of 16), into dst[4] at slot * dst_stride[s]
 * bytes; the scales are converted to scale_dt.  max_copies = n_pairs.  No
 * host synchronisation: a paged step can be captured in a HIP graph.
 * Replaces the host LRU and synchronous per-slot copies of
 * PagedMoEExpert._get_slot / forward (vq2/paged_runtime.py:415-437, 491-500). */
size_t vq2_pager_lds_bytes(int64_t n_experts, int64_t capacity, int64_t n_pairs);
int vq2_pager_step(const void* ids, int ids_i64, int64_t n_pairs, int64_t n_experts, int64_t capacity,
                   int32_t* slot_of, int32_t* expert_of, int32_t* stamp, int32_t* state, int32_t* copy_list,
                   int32_t* pair_slot, void* stream);
int vq2_pager_copy(const void* mirror, int64_t record_bytes, const int64_t* seg_bytes, const int32_t* copy_list,
                   const int32_t* state, int64_t max_copies, void* const* dst, const int64_t* dst_stride, int scale_dt,
                   void* stream);

/* Rotated-space dequantisation of rows [r0, r1) (debug / audit):
 *   W[r, 8g+j] = (f32(cb0[i0]) [+ f32(cb1[i1])]) * f32(scale[r]), fp32 [r1-r0, n]
 * rounded exactly in that order (no contraction).
 * Replaces QMat.dequant before rot.inv (vq2/vq.py:283-292) and
 * PackedLinear.weight_rows in fp32 (vq2/runtime.py:82-89). */
int vq2_dequant_rows(const int16_t* idx0, const void* idx1, int s2_kind,
                     const void* cb0, const void* cb1, int cb_dt,
                     const void* scale, int s_dt,
                     int64_t r0, int64_t r1, int64_t n, float* out, void* stream);

/* Index decode: out[i] = (int32)in[i] & 0xFFFF (int16 planes) or the byte
 * value (uint8 planes, is_u8 != 0).  Replaces _as_index (vq2/runtime.py:32-35). */
int vq2_decode_idx(const void* in, int is_u8, int64_t count, int32_t* out, void* stream);

/* Fixed-width symbol stream -> uint16 codes (int16 storage, the planes the
 * GEMV reads): n symbols of bits in {4, 8, 12, 16} from nbytes >=
 * ceil(n * bits / 8) bytes, in the little-endian packing of
 * vq2/export.py:39-53 (pack_fixed).  Replaces unpack_fixed
 * (vq2/export.py:56-70) at container load time. */
int vq2_unpack_fixed(const uint8_t* buf, int64_t nbytes, int bits, int64_t n, int16_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VQ2_AMD_H */
