/* exl3mi: EXL3 trellis-quantized linear and grouped-MoE kernels for AMD Instinct MI355X (gfx950).
 *
 * Plain C ABI: device pointers, sizes, a hipStream_t passed as void*. Every entry point is asynchronous on `stream`
 * (NULL = the default stream), never synchronises the host (the workspace calls below say where they do), and
 * returns an exl3_status. The caller owns every input and output buffer; outputs are written in place.
 * Library-owned scratch is cached per device (grown on demand; see exl3_reserve_workspace). Calls on one device must
 * be ordered on one stream: they share that device's workspace, and two calls that overlap in time race on it.
 *
 * Data formats (identical to exllamav3 / the reference, ext-op-inventory.md:698-777):
 *   trellis  int16 [k/16][n/16][16*K], K = bits per weight (1..8), one 16x16 tile = 8*K little-endian uint32 words
 *   suh      fp16 [k], svh fp16 [n] (sign flips with the channel scales folded in)
 *   W = diag(suh) Hblk W_hat Hblk diag(svh), Hblk = blockdiag(H128 / sqrt(128)); y = x @ W
 * Codebook: only cb = 2 (mul1, the codebook every checkpoint of the reference uses) is implemented.
 */
#ifndef EXL3MI_H
#define EXL3MI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_ABI_VERSION 2

enum exl3_status {
    EXL3_OK = 0,
    EXL3_ERR_INVALID = 1,     /* bad shape, dtype, alignment or pointer: the reference's TORCH_CHECK -> RuntimeError */
    EXL3_ERR_UNSUPPORTED = 2, /* K / codebook / mode not implemented: NotImplementedError */
    EXL3_ERR_HIP = 3          /* HIP runtime error */
};

enum exl3_dtype { EXL3_F16 = 0, EXL3_F32 = 1 };
enum exl3_act { EXL3_ACT_SILU = 0, EXL3_ACT_GELU_TANH = 1 };
enum exl3_score { EXL3_SCORE_SOFTMAX = 0, EXL3_SCORE_SIGMOID = 1, EXL3_SCORE_SQRT_SOFTPLUS = 2 };
enum exl3_route_flags { EXL3_ROUTE_RENORM = 1, EXL3_ROUTE_BIAS_SELECT_ONLY = 2 };
enum exl3_router_w { EXL3_ROUTER_W_HE = 0, EXL3_ROUTER_W_EH = 1 };
enum exl3_word_order { EXL3_WORDS_PLANAR4 = 0, EXL3_WORDS_TILE_ORDER = 1 };

/* Message for the last non-zero status returned on the calling thread. */
const char* exl3_last_error(void);
int exl3_abi_version(void);

/* Pre-size this device's workspace (bytes of scratch, number of arrival counters) so later calls do not allocate,
 * e.g. before HIP graph capture (a call that would grow the workspace while its stream is being captured fails with
 * EXL3_ERR_INVALID). Synchronises the device. Growing (here or inside a call) keeps the outgrown buffers alive, since
 * queued kernels and captured graphs may still use them, until exl3_release_workspace.
 * No reference counterpart (the reference grows its scratch inside the op, glm/xpu/csrc/exl3_ops.sycl:202-207). */
int exl3_reserve_workspace(int64_t bytes, int64_t ncounters);

/* Free the outgrown workspace buffers of the current device. Synchronises the device; graphs captured while those
 * buffers were current must not be replayed afterwards. No reference counterpart. */
int exl3_release_workspace(void);

/* The current device's status word: 0, or 1 after a fused MoE layer launch or a one-row decode GEMV launch of
 * exl3_gemm / exl3_linear_sharded (whose last k-split waits for the other splits' partials) gave up one of its bounded
 * cross-workgroup waits (its outputs, and possibly those of launches queued behind it, are then incomplete). Read on
 * the host without synchronising. The next library call on the device that uses the workspace outside stream capture
 * zeroes every arrival-counter buffer of the device on its stream (the current one and the outgrown ones that graphs
 * captured earlier still use), clears the word and returns EXL3_ERR_HIP; a call under capture returns EXL3_ERR_HIP and
 * leaves the word set. Graph replays do not check the word: code that replays graphs polls it and, when set, makes
 * one eager call that takes the workspace (exl3_reserve_workspace(0, 0)) to reset. No reference counterpart (the
 * reference's kernels do not wait across work-groups). */
int exl3_device_status(int* status);

/* Kernel timing: while enabled (on != 0), every kernel the library launches is bracketed by a HIP event pair on its
 * stream; with on = R > 1 each launch runs R times inside its pair (the kernels are idempotent) to amortise the event
 * overhead. exl3_profile_read writes "name count avg_us" lines (per-launch averages) since the last enable.
 * Not for use under graph capture. No reference counterpart (the reference times with torch.profiler). */
int exl3_profile_enable(int on);
int exl3_profile_read(char* out, int64_t cap);

/* Decoded Hadamard-domain weight slice: out[r, c] = W_hat[r, n_offset + c] (fp16 bits, row stride out_ld elements),
 * no sign vectors applied. Bit-exact with the reference decode.
 * Replaces: exllamav3 ext reconstruct / reconstruct_slice (ext-op-inventory.md:597-612) and
 *           exl3xpu_C::exl3_reconstruct (glm/xpu/csrc/exl3_ops.sycl:539-555, bound at :791-799).
 * k % 16 == 0, n_total % 16 == 0, n_offset and n_slice multiples of 128, n_offset + n_slice <= n_total. */
int exl3_reconstruct(const int16_t* trellis, int64_t k, int64_t n_total, int K, int cb, int64_t n_offset,
                     int64_t n_slice, uint16_t* out, int64_t out_ld, void* stream);

/* Original-basis weight slice: out[r, c] = W[r, n_offset + c] with W = diag(suh) Hblk W_hat Hblk diag(svh_full),
 * where svh points at the slice's output signs (svh_full + n_offset, as the reference passes svh[n_start:]) and suh
 * covers all k rows; fp16 out (row stride out_ld), computed in fp32 and rounded once (within one fp16 rounding of the
 * exact weight; the reference's fp16 butterflies are less precise, so results are not bit-identical with it).
 * y = x @ out is the linear's output for those columns. k, n_total, n_offset and n_slice multiples of 128.
 * Replaces: exllamav3 ext reconstruct_had_slice(unpacked, packed, suh, svh, K, mcg, mul1, n_offset)
 *           (ext-op-inventory.md:614-627; the fused large-M prefill, ext-op-inventory.md:437-446). */
int exl3_reconstruct_had_slice(const int16_t* trellis, int64_t k, int64_t n_total, int K, int cb, const uint16_t* suh,
                               const uint16_t* svh, int64_t n_offset, int64_t n_slice, uint16_t* out, int64_t out_ld,
                               void* stream);

/* Blockwise 128-point Hadamard: out[r, blk] = (H128 @ (in[r, blk] (* pre))) * scale / sqrt(128) (* post).
 * in/out [rows, cols] with row strides in_ld/out_ld, both of `dtype`; cols % 128 == 0; in-place allowed.
 * pre/post fp16 [cols] or NULL; if both are given only pre is applied. fp16 path rounds x*pre, the scaled sum and
 * the *post product to fp16; the fp32 path does not round.
 * Replaces: exllamav3 ext had_r_128 (ext-op-inventory.md:576-595; glm/xpu/glm_xpu/ops.py:130-142). */
int exl3_had_r_128(const void* in, int64_t in_ld, void* out, int64_t out_ld, int64_t rows, int64_t cols, int dtype,
                   const uint16_t* pre, const uint16_t* post, float scale, void* stream);

/* EXL3 linear: C[m, n] = Hn( Hk(A * suh) @ W_hat ) * svh for A fp16 [m, k] (row stride a_ld), C fp16 or fp32
 * [m, n] (row stride c_ld). A_had (fp16 scratch, >= m*k elements) is accepted for signature compatibility and not
 * used: the input transform is fused. cb must be 2 (mul1). Up to 8 rows: decode GEMV (at one row the last k-split
 * waits, bounded, for the others' partials: exl3_device_status); 9 rows and more: the trellis
 * decoded into fp16 MFMA fragments once per row block of up to 64 rows (the reference's large-M linear,
 * exl3_ops.sycl:742-756, reconstructs fp16 slices and calls a GEMM instead; same results within the tolerance).
 * Replaces: exllamav3 ext exl3_gemm(A, B, C, suh, A_had, svh, force_shape_idx, mcg, mul1, force_num_sms)
 *           (ext-op-inventory.md:498-557) and exl3xpu_C::exl3_gemm_small / linear (glm/xpu/csrc/exl3_ops.sycl:258-321,
 *           643-757). */
int exl3_gemm(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K, void* C,
              int64_t c_ld, int c_dtype, const uint16_t* suh, uint16_t* A_had, const uint16_t* svh, int cb,
              void* stream);

/* exl3_gemm for up to 8 rows (the decode GEMV, same kernels and results bit for bit) without the library workspace:
 * its split-K partials and arrival counters live in a fixed device array (16 MiB + 64 KiB per device, held until the
 * process ends), so the call never allocates, e.g. under HIP graph capture or in a serving loop that must not
 * allocate. Limits: m <= 8, n <= 2 097 152 columns, and strips (n / 128) x k-splits x 8 x 128 x 4 bytes of partials
 * <= 16 MiB (k-splits <= 16; e.g. n = 21504 at any k fits); larger shapes return EXL3_ERR_INVALID. Every call on a
 * device shares that device's array: calls that overlap in time (two streams, two threads) race. A_had is dropped.
 * No counterpart in the reference: an entry point for callers that cannot allocate. */
int exl3_gemm_noalloc(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K,
                      void* C, int64_t c_ld, int c_dtype, const uint16_t* suh, const uint16_t* svh, int cb,
                      void* stream);

/* Fused multi-projection linear: S projections that share the input x (e.g. q|k|v or gate|up), their trellises
 * concatenated along the output columns (B = [k/16][n/16][16K] with n = the sum of the projections' widths, as
 * torch.cat(trellises, 1)), per-projection input signs suh fp16 [S][k] (row s for shard s), output signs svh fp16 [n]
 * (concatenated), and shard_of_nb int32 [n/128] (device) naming the shard of every 128-column block (values outside
 * [0, S) are clamped). Column block j of C is x @ W_{shard_of_nb[j]} for that block. n_shards = 1 (shard_of_nb may be
 * NULL) is exl3_gemm. Other arguments and paths as exl3_gemm.
 * Replaces: exl3xpu_C::linear(x, trellis, suh[S, k], svh[n], shard_of_nb, group_bounds, K, cb, small_m_max, slice_n)
 *           (glm/xpu/csrc/exl3_ops.sycl:651-757, bound at :789-790) and exl3_gemm_small with shard_of_nb (:258-321). */
int exl3_linear_sharded(const uint16_t* A, int64_t a_ld, int64_t m, int64_t k, const int16_t* B, int64_t n, int K,
                        void* C, int64_t c_ld, int c_dtype, const uint16_t* suh, int64_t n_shards,
                        const int32_t* shard_of_nb, const uint16_t* svh, int cb, void* stream);

/* Multi-matrix EXL3 linear over `slots` slots. Matrix q (0 <= q < num_mats) is the trellis, suh and svh whose device
 * addresses are B_ptrs[q], suh_ptrs[q], svh_ptrs[q] (int64 device tables; every matrix [k, n] at bitrate K, trellis
 * 4-byte aligned). Slot j runs matrix q_j = indices[j] (int64 device array, or j when indices is NULL); with
 * min_index >= 0 only q in [min_index, max_index) run, as q - min_index; slots whose q is negative or not below
 * num_mats are skipped. Slot j reads A batch 0 (a_batches == 1), j (a_batches == slots) or j / (slots / num_tokens)
 * (a_batches == num_tokens) of A fp16 [a_batches, m, k] (contiguous) and computes Y_j = exl3_gemm(A_batch, q_j), [m, n].
 * Without weights: C[j] = Y_j, C [slots, m, n] (fp16 or fp32, contiguous); skipped slots leave C[j] unchanged.
 * With weights (fp16 [slots], device): C[t] = sum over token t's slots j = t * (slots / num_tokens) + i in order of
 * weights[j] * Y_j (fp32 sum, one rounding for fp16 C; skipped slots add nothing), C [num_tokens, m, n]. Rows are
 * processed 8 at a time by the decode GEMV (the op serves decode batches). cb must be 2 (mul1). Differences from the
 * reference op: for fp16 C it adds each slot's fp16 result with __hadd (ext-op-inventory.md:682), this sums in
 * fp32 and rounds once (a few fp16 ulps apart at most); it returns the shape index it ran, this returns a status.
 * Replaces: exllamav3 ext exl3_mgemm(A, B, C, suh, A_had, svh, indices, weights, K, force_shape_idx, mcg, mul1,
 *           min_index, max_index, force_num_sms, num_tokens, ...) (ext-op-inventory.md:664-685, 1104-1119); the
 *           sliced mode (size_n_list, c_ptrs, n_stride_list, had_src_list) is not provided. */
int exl3_mgemm(const uint16_t* A, int64_t a_batches, int64_t m, int64_t k, const int64_t* B_ptrs,
               const int64_t* suh_ptrs, const int64_t* svh_ptrs, int64_t num_mats, int64_t n, int K, int cb,
               const int64_t* indices, int64_t slots, const uint16_t* weights, int64_t num_tokens, int64_t min_index,
               int64_t max_index, void* C, int c_dtype, void* stream);

/* Gated activation z = act(x, y) elementwise over n values, fp16 (dtype EXL3_F16) or fp32 (EXL3_F32) inputs, fp16
 * output (in place on y allowed). SiLU: z = min(silu(x), L) * clamp(y, -L, L) (L = act_limit, 0 disables);
 * GELU-tanh: z = gelu_tanh(x) * y. Computed in fp32, rounded once.
 * Replaces: exllamav3 ext silu_mul / gelu_mul (ext-op-inventory.md:944-956; glm/xpu/glm_xpu/ops.py:147-154). */
int exl3_act_mul(const void* x, const void* y, uint16_t* z, int64_t n, int dtype, int act, float act_limit,
                 void* stream);

/* ---------------------------------------------------------------------------------------------- grouped MoE
 * Expert tables: `tables` is a device int64 array [9][E] of device addresses, row 3p + {0, 1, 2} = (trellis, suh,
 * svh) of projection p = 0 gate [H -> I], 1 up [H -> I], 2 down [I -> H], the nine per-projection pointer tables of
 * the reference's BC_BlockSparseMLP / exl3_moe (ext-op-inventory.md:1027-1034, 1060-1093).
 * K_gate / K_up / K_down: bits per weight of each projection (1..8, gate and up equal), or 0 = per-tile K: then
 * `kmaps` (device int64 [6][E]) holds for projection p the address of a uint8 [k/16 * n/16] tile-K map (row-major
 * tiles) at row 2p and of an int32 [k/16 * n/16 + 1] word-offset prefix at row 2p + 1; the trellis address is the
 * base of the concatenated tile words (tile i: 8 * kmap[i] words at offset woff[i]). kmaps may be NULL otherwise. */

/* Routed MoE layer: out[t] = sum_{j < topk, slot order} w[t, j] * expert_{ids[t, j]}(x[t]) (+ expert `shared`(x[t])
 * with weight 1 after the routed slots when shared >= 0). expert(x) = down(act(gate(x), up(x))) with the reference
 * rounding points: gate/up outputs fp16, activation fp16, down input transform fp16, fp32 accumulation.
 * x fp16 [M, H] (row stride x_ld); topk_ids int32 [M, topk] in [0, E) (negative = inactive slot); topk_w fp32
 * [M, topk]; out fp32 or fp16 [M, H] (row stride out_ld). H % 128 == 0, I % 128 == 0.
 * act: EXL3_ACT_SILU (a = min(silu(g), L) * clamp(u, -L, L), L = act_limit, 0 = no clamp) or EXL3_ACT_GELU_TANH.
 * Batches of at most 16 tokens and 128 (token, slot) pairs run as one fused launch; larger batches on 8 tokens or
 * fewer use the decode GEMV kernels, and larger ones the fp16 MFMA grouped GEMM.
 * Replaces: BC_BlockSparseMLP.run_bszN and exl3_moe + exl3_moe_gather over the nine pointer tables
 *           (ext-op-inventory.md:1036-1102), dsv_moe::moe_gemv with per-item K (dsv41/xpu/csrc/dsv_moe.sycl:157-170).
 *           The reference's blob-pointer op is exl3_moe_forward_blobs below. */
int exl3_moe_forward(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, const int32_t* topk_ids,
                     const float* topk_w, int64_t topk, int64_t E, const int64_t* tables, const int64_t* kmaps,
                     int K_gate, int K_up, int K_down, int act, float act_limit, int64_t shared, void* out,
                     int64_t out_ld, int out_dtype, void* stream);

/* The routed MoE layer over the reference's expert blobs: ptrs (device int64 [E]) holds one blob address per expert,
 * each blob laid out as the reference's Geom (glm/xpu/csrc/exl3_moe.n128.sycl:3-11, 56-68; packed by pack_expert,
 * glm/xpu/exl3xpu/moe_offload.py:81-94): gate|up trellis uint32 [H/16][2I/16][8K] (per tile-row the I/16 gate tiles,
 * then the I/16 up tiles), down trellis [I/16][H/16][8K], then fp16 suh_g[H] suh_u[H] svh_g[I] svh_u[I] suh_d[I]
 * svh_d[H]; blobs 16-byte aligned, every routed expert's pointer valid. word_order EXL3_WORDS_PLANAR4: the trellis
 * words as the reference packs them and its kernels read them, in place (PLANAR4: a tile's 8K words are G periods
 * of D = K / gcd(K, 32) words, and within each group of 4 consecutive tiles of a tile-row word (tile t, period g,
 * plane i) sits at 4G i + G t + g, G = 8K / D; for K = 1, 2, 4, 8 that is tile order; glm/xpu/exl3xpu/
 * moe_offload.py:68-78, glm/xpu/pack_store.py:35-54). EXL3_WORDS_TILE_ORDER: blobs that exl3_blob_unplanarize has
 * converted (every K; the same words at even K). One K for all projections, 1..8 (the reference op takes 2, 3 and 4);
 * no shared expert (the reference adds it outside the op). Other arguments, paths and results as exl3_moe_forward
 * with the same weights.
 * Replaces: exl3xpu_moe::moe_forward(x, topk_ids, topk_w, ptrs, I, K, n_experts) (glm/xpu/csrc/exl3_moe.n128.sycl:
 *           1380-1439, bound at :1681-1682). */
int exl3_moe_forward_blobs(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, const int32_t* topk_ids,
                           const float* topk_w, int64_t topk, int64_t E, const int64_t* ptrs, int K, int act,
                           float act_limit, void* out, int64_t out_ld, int out_dtype, int word_order, void* stream);

/* Optional one-time conversion of the reference's expert blobs to tile order, in place: where PLANAR4 differs from
 * tile order (K = 3, 5, 6, 7) the words of every group of 4 tiles of a tile-row are put back into tile order; other K
 * need no work. Blobs and sizes as exl3_moe_forward_blobs. Afterwards the blobs are read with EXL3_WORDS_TILE_ORDER
 * (one K-dword load per lane instead of K dword loads) and no longer serve the reference's kernels; converting a blob
 * twice scrambles it.
 * No reference counterpart: the reference's kernels always read PLANAR4 (Xe register regions cannot stride by K). */
int exl3_blob_unplanarize(const int64_t* ptrs, int64_t E, int64_t H, int64_t I, int K, void* stream);

/* The routed MoE layer from router logits: exl3_route_softmax_topk followed by exl3_moe_forward, as one call, with
 * the same results bit for bit. Up to 2 tokens with n_logits <= 512 on the fused decode layer, the layer ranks the
 * logits itself (one launch); otherwise the routing launch runs first on the same stream. logits fp32 [M, n_logits]
 * (row stride logits_ld),
 * bias fp32 [n_logits] or NULL; the routed experts are table entries 0 .. n_logits - 1 (n_logits <= E; the shared
 * expert, if any, is another entry). ids_out int32 [M, topk] and w_out fp32 [M, topk] receive the routing.
 * topk <= 32, n_logits <= 8192. table_layout: NULL, or a HOST array of 18 int64 (base[9], stride[9]) with
 * tables[i][e] == base[i] + e * stride[i] for every expert e < E (experts packed at uniform strides, as
 * ExpertTables.packed builds them): the decode kernels then compute an expert's addresses instead of loading them.
 * Replaces: the router + BlockSparseMLP.forward pair (glm/xpu/glm_xpu/moe_patch.py:68-94 with the trellis-serve fused
 * router, trellis-serve.patch:395-441). */
int exl3_moe_forward_logits(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, int64_t I, const float* logits,
                            int64_t logits_ld, int64_t n_logits, const float* bias, int64_t topk, int64_t E,
                            const int64_t* tables, const int64_t* kmaps, int K_gate, int K_up, int K_down, int act,
                            float act_limit, int64_t shared, const int64_t* table_layout, int32_t* ids_out,
                            float* w_out, void* out, int64_t out_ld, int out_dtype, void* stream);

/* Routing tables as the MoE kernels build them (pairs grouped by expert), for tests and debugging.
 * Writes counts int32 [E], pair_tok int32 [M*slots], pair_w fp32 [M*slots], pair_of int32 [M*slots]
 * (slots = topk + (shared >= 0)); pair order inside an expert is unspecified.
 * Replaces: exl3xpu_moe::moe_align (glm/xpu/csrc/exl3_moe.n128.sycl:1441-1448). */
int exl3_moe_align(const int32_t* topk_ids, const float* topk_w, int64_t M, int64_t topk, int64_t E, int64_t shared,
                   int32_t* counts, int32_t* pair_tok, float* pair_w, int32_t* pair_of, void* stream);

/* Softmax router: p = softmax(logits + bias) over E experts, top-k by p (ties to the lower index, descending),
 * weights renormalised over the k picks with +1e-20. logits fp32 [M, E] (row stride ld), bias fp32 [E] or NULL;
 * ids int32 [M, k], w fp32 [M, k]. k <= 32, E <= 8192. Same as exl3_route_topk(..., EXL3_SCORE_SOFTMAX,
 * EXL3_ROUTE_RENORM, 1.0f, ...).
 * Replaces: the fused softmax/top-k router of trellis-serve (trellis-serve.patch:395-441). */
int exl3_route_softmax_topk(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, int64_t k,
                            int32_t* ids, float* w, void* stream);

/* Top-k router with a choice of scoring, one row per wave. Per expert e with logit f and bias b (bias NULL: b = 0):
 *   EXL3_SCORE_SOFTMAX        rank by f + b; weights from p = softmax(f + b), or softmax(f) with
 *                             EXL3_ROUTE_BIAS_SELECT_ONLY (the bias only ranks: trellis-serve's `cold` term)
 *   EXL3_SCORE_SIGMOID        s = sigmoid(f); rank by s + b (by f without a bias); weights from s
 *   EXL3_SCORE_SQRT_SOFTPLUS  s = sqrt(softplus(f)) (softplus(f) = f above 20); rank by s + b; weights from s
 * Picks in descending rank order, exact ties to the lower index. Weight of a pick: v * scaling / (sum of the picks'
 * v + 1e-20) with EXL3_ROUTE_RENORM, v * scaling without. Sizes as exl3_route_softmax_topk.
 * Replaces: routing_ds3_nogroup's selection and weights (glm/xpu/glm_xpu/ops.py:177-193), the dsv Route kernel
 * (dsv41/xpu/csrc/dsv_moe_glue.sycl:155-193, without its residency terms), trellis-serve's router with `cold`
 * (trellis-serve.patch:395-441). */
int exl3_route_topk(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, int64_t k, int score,
                    int flags, float scaling, int32_t* ids, float* w, void* stream);

/* Top-k routing with the reference dsv router's residency terms: the picks rank by s * mul[e] + bias[e] +
 * max(res[e], -1e30) (s = sigmoid or sqrt-softplus of the logit, each operation rounded separately; mul, res fp32 [E]
 * or NULL: a per-expert selection multiplier and an additive 0 / -margin / -inf residency bias, so that experts
 * already in memory are preferred), exact ties to the lower index; the weights come from s as in exl3_route_topk
 * (flags: EXL3_ROUTE_RENORM). E <= 2048. The plain picks (the reference's `want`) are exl3_route_topk with the same
 * bias.
 * Replaces: dsv_moe::moe_route(logits, bias, res, ids, w, want, scaling) and the mul term of route_fused
 *           (dsv41/xpu/csrc/dsv_moe_glue.sycl:155-193, 426-439, bound at :621-622). */
int exl3_route_adjusted(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, const float* mul,
                        const float* res, int64_t k, int score, int flags, float scaling, int32_t* ids, float* w,
                        void* stream);

/* Verify-block routing (sqrt-softplus): rows in blocks of rows_per_block (M a multiple), each block's rows in order; an
 * expert that an earlier row of the block picked ranks by s * mul[e] * (1 + block_boost) + bias[e], the others by
 * s * mul[e] + bias[e] (mul, bias fp32 [E] or NULL; each operation rounded separately), exact ties to the lower
 * index; weights s renormalised (+1e-20) * scaling. E <= 2048, k <= 32.
 * Replaces: the block mode of dsv_moe::route_fused (RouteBlock, dsv41/xpu/csrc/dsv_moe_glue.sycl:194-240, 495-507). */
int exl3_route_block(const float* logits, int64_t ld, int64_t M, int64_t E, const float* bias, const float* mul,
                     int64_t k, int64_t rows_per_block, float block_boost, float scaling, int32_t* ids, float* w,
                     void* stream);

/* Router logits from hidden states: logits[m, e] = sum_h x[m, h] * W(h, e) in fp32 (fixed summation order), x fp16
 * [M, H] (row stride x_ld), logits fp32 [M, E] (row stride logits_ld), rounded to fp16 precision when round_fp16 != 0
 * (what a matmul of two fp16 tensors returns). w_layout EXL3_ROUTER_W_HE: W fp16 [H, E] (row stride w_ld >= E,
 * E % 8 == 0: the reference's gate_tensor[:, :E]); EXL3_ROUTER_W_EH: W fp16 [E, H] (row stride w_ld >= H, a linear
 * layer's weight). H % 128 == 0; W 16-byte aligned, w_ld % 8 == 0.
 * Replaces: torch.matmul(hidden, gate[:, :E]) of routing_ds3_nogroup (glm/xpu/glm_xpu/ops.py:183-184) and the GemvH
 * router GEMV of route_fused / gemv_h (dsv41/xpu/csrc/dsv_moe_glue.sycl:442-470, 520-530). */
int exl3_router_logits(const uint16_t* x, int64_t x_ld, int64_t M, int64_t H, const uint16_t* W, int64_t w_ld,
                       int64_t E, int w_layout, int round_fp16, float* logits, int64_t logits_ld, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3MI_H */
