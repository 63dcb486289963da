/*
 * quail_mi355x.h - C ABI of libquail_mi355x.so, the gfx950 (MI355X) kernels
 * of Quail's packed-prompt prefill pass for Qwen3 FP8 models.
 *
 * Each entry point replaces one call on the reference's hot path; the
 * comment above it cites the reference interface (paths relative to the
 * fsdatalab/quail repository) whose result it reproduces.
 *
 * Conventions
 *   - Pointers are device pointers; sizes and strides are int64 and count
 *     elements of the pointed-to type (bytes for e4m3 data).
 *   - Work is enqueued on `stream` and never synchronized; the caller keeps
 *     every buffer alive until the stream has passed the call.
 *   - bf16 is passed as raw 16-bit words; e4m3 as OCP e4m3fn bytes (max 448).
 *   - FP8 activation scales are "column-major": the scale of token t and
 *     128-column group g is at scales[g * s_ld + t] (attention.py:534-537).
 *   - Return value: 0 on success; -1 for an argument error, with the
 *     message in qx_last_error(); a positive hipError_t if the launch failed.
 *   - The device entry points allocate no memory and keep no state between
 *     calls; the host packing functions (qx_pages_*, qx_pack_*) keep theirs
 *     in host handles the caller creates and destroys.
 */
#ifndef QUAIL_MI355X_H
#define QUAIL_MI355X_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * ABI version of the library: qx_version() returns the QX_ABI_VERSION it
 * was built with. It is raised whenever an entry point changes its
 * arguments or their meaning, so that a caller built against another
 * header fails at load time instead of passing arguments in the wrong
 * slots. 1: the first release. 2: qx_paged_attention and
 * qx_paged_attention_work take tile_rows, qx_paged_attention and
 * qx_attention_lse take v_bf16, qx_qk_norm_rope_kv takes v_f16.
 */
#define QX_ABI_VERSION 2
int qx_version(void);

/* Text of the last argument error on the calling thread. */
const char* qx_last_error(void);

/* 1 if the current HIP device is gfx950, 0 if not, <0 on a HIP error. */
int qx_device_is_gfx950(void);

/*
 * FP8 block-scaled GEMM, bf16 output:
 *   C[m,n] = sum_kb sA[kb*sa_ld + m] * sW[(n/128)*(K/128) + kb] * sum_{k in kb} A[m,k] W[n,k]
 * Replaces Engine.gemm -> DeepGEMM fp8_gemm_nt((A, sA), (W, sW), C)
 * (quail/backends/quail/executor/attention.py:479-490); weight scales are the
 * checkpoint's weight_scale_inv (attention.py:471-477).
 * K and N multiples of 128. config selects the tile shape, tokens x weights,
 * all with two pipeline stages of one 128-K scale block each:
 * 10: 256x256 tiles, 8 waves, one workgroup per tile (N a multiple of 256);
 * 11: 256x128 tiles, 4 waves (any N);
 * 12: 256x320 tiles, 8 waves (N a multiple of 320: whole waves of tiles on
 *     256 CUs where N = 2560 and M is a multiple of 8192 or just under one);
 * 22: 256x256 tiles walked by one persistent workgroup per CU, the next
 *     tile's first block loaded during the last block of the current one
 *     and the epilogue staged in two passes through one stage buffer (falls
 *     back to 10 with an odd number of 128-K blocks or too few tiles);
 * 30: the promotion form (DeepGEMM's arithmetic): each 128-K block's
 *     products summed from zero by one 16x16x128 MFMA per 16x16 output
 *     tile, then total += (sA * sW) * partial in fp32; 256x256 tiles on a
 *     persistent grid, the next block's loads issued one per MFMA (N a
 *     multiple of 256; any number of 128-K blocks);
 * 31: config 30's arithmetic on 256x320 tiles (N a multiple of 320): each
 *     wave's 160 weight rows lie in two 128-row scale blocks and each of
 *     its 16-row tiles is promoted with its block's scale; bit-identical
 *     to config 30 where N is a multiple of both.
 * Configs 10, 11, 12 and 22 rescale the accumulators in place
 * (acc *= s_prev / s per block, the last s in the epilogue) and compute
 * each element with the same operations in the same order: their results
 * are bit-identical for finite operands. A weight block whose scale is 0
 * is skipped by 10, 11 and 22 and run on zeroed weight rows by 12, so a
 * NaN activation code in such a block gives 0 under 10/11/22 and NaN under
 * 12; configs 30 and 31 add 0 * partial, NaN as well, as DeepGEMM's
 * promotion does. Configs 30 and 31 sum in another order (within the bf16
 * tolerance of the others and of the dequantized product); a caller that
 * needs a row's result independent of M picks the family by N alone.
 */
int qx_gemm_fp8_blockscaled(const void* A, const float* sA, const void* W, const float* sW,
                            void* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldc,
                            int64_t sa_ld, int config, hipStream_t stream);

/*
 * res <- bf16(x + res); y = (x + res) * rsqrt(mean((x+res)^2) + eps) * w in
 * fp32; per-token 128-group e4m3 quant of y with scale max(amax,1e-10)/448.
 * Replaces the Triton add_rms_norm_quant (attention.py:796-829) called from
 * Engine.custom_norm_quant (attention.py:1098-1111).
 */
int qx_add_rmsnorm_quant(const void* x, int64_t x_ld, void* res, int64_t res_ld, const void* w,
                         void* q, int64_t q_ld, float* scales, int64_t s_ld, int64_t n, int64_t H,
                         float eps, hipStream_t stream);

/*
 * y = bf16(bf16(x * rstd) * w), then per-token 128-group e4m3 quant.
 * Replaces Engine.norm_quant without a residual: vLLM rms_norm then
 * per_token_group_quant_fp8 (attention.py:1237-1240, 539-556, 517-532).
 */
int qx_rmsnorm_quant(const void* x, int64_t x_ld, const void* w, void* q, int64_t q_ld,
                     float* scales, int64_t s_ld, int64_t n, int64_t H, float eps,
                     hipStream_t stream);

/*
 * res[i] = table[ids[i]] (bf16), then qx_rmsnorm_quant of that row: the
 * embedding gather of Qwen3Pipeline.forward_chunk (qwen3.py:123) fused with
 * layer 0's norm_quant (qwen3.py:47-49).
 */
int qx_embed_rmsnorm_quant(const void* table, int64_t t_ld, const int64_t* ids, void* res,
                           int64_t res_ld, const void* w, void* q, int64_t q_ld, float* scales,
                           int64_t s_ld, int64_t n, int64_t H, float eps, hipStream_t stream);

/*
 * vLLM fused_add_rms_norm (attention.py:558-562): z = bf16(h + r);
 * res_out <- z; out = bf16(bf16(z * rstd) * w). With rows != NULL, output
 * row i reads input row rows[i] (the final_indices gather of qwen3.py:130-134).
 * out may alias h and res_out may alias r only when rows == NULL.
 */
int qx_add_rmsnorm(const void* h, int64_t h_ld, const void* r, int64_t r_ld, const int64_t* rows,
                   const void* w, void* out, int64_t out_ld, void* res_out, int64_t res_out_ld,
                   int64_t n, int64_t H, float eps, hipStream_t stream);

/*
 * Per-head RMSNorm of q (HQ heads) and k (HK heads) of the fused qkv rows,
 * then neox RoPE from cos_sin[positions[i]] = [cos D/2 | sin D/2], fp32
 * math, bf16 outputs. Replaces the Triton qk_norm_rope (attention.py:833-879)
 * called from Engine.custom_qk_norm_rope (attention.py:1113-1128).
 * cs_is_f32 selects an fp32 cache; otherwise it is bf16.
 */
int qx_qk_norm_rope(const void* qkv, int64_t qkv_ld, void* q_out, int64_t q_ld, void* k_out,
                    int64_t k_ld, const void* cos_sin, int cs_is_f32, const int64_t* positions,
                    const void* q_w, const void* k_w, int64_t n, int64_t HQ, int64_t HK,
                    int64_t D, float eps, hipStream_t stream);

/*
 * qx_qk_norm_rope with the row's KV written straight into arena pages: q as
 * above (q_out may be NULL: then only K and V are written, for
 * qx_paged_attention_qnorm, which normalizes and rotates q itself); the
 * normed, rotated K of row i goes to pool row dst[i] of k_pool and
 * its V (qkv columns (HQ+HK)*D .. (HQ+2*HK)*D, bf16) to the same row of
 * v_pool, as bf16, or with v_f16 as fp16 (round to nearest even, saturated
 * at +-65504); dst[i] < 0 writes neither. Pool rows are HK*D
 * elements. dst2 (may be NULL): the same K and V rows also go to row
 * dst2[i] (when >= 0) of k_pool2 / v_pool2 (the tree path: contiguous rows
 * for call A, dst = 0..n-1, and the arena pages). The same values as
 * qx_qk_norm_rope followed by qx_kv_scatter (src = 0..n-1), in
 * one pass over qkv: it fuses Engine.qk_norm_rope (attention.py:1251-1255)
 * with the fresh-row write of Engine.write_kv (attention.py:1178-1191) when
 * the pack's scatter source is its own rows in order; the retained-tail copy
 * stays a qx_kv_scatter.
 */
int qx_qk_norm_rope_kv(const void* qkv, int64_t qkv_ld, void* q_out, int64_t q_ld, void* k_pool,
                       void* v_pool, const int64_t* dst, void* k_pool2, void* v_pool2,
                       const int64_t* dst2, const void* cos_sin, int cs_is_f32,
                       const int64_t* positions, const void* q_w, const void* k_w, int64_t n,
                       int64_t HQ, int64_t HK, int64_t D, float eps, int v_f16,
                       hipStream_t stream);

/*
 * y = g * sigmoid(g) * u over rows [g (I) | u (I)], fp32; per-token
 * 128-group e4m3 quant. Replaces the Triton silu_mul_quant
 * (attention.py:771-793) called from Engine.custom_silu_quant (:1084-1096).
 */
int qx_silu_mul_quant(const void* gate_up, int64_t gu_ld, void* q, int64_t q_ld, float* scales,
                      int64_t s_ld, int64_t n, int64_t I, hipStream_t stream);

/*
 * The gate_up projection and the SiLU-gated product with its per-token
 * 128-group e4m3 quant in one launch: replaces the pair
 * Engine.gemm(g_in, g_scale, mlp.gate_up_proj) (attention.py:479-490) +
 * Engine.activation_quant (attention.py:1245-1249 -> :771-793) that
 * qwen3.py:66-67 issues. W / sW are the checkpoint's gate_up weight
 * (2I x K, rows [gate | up]) and weight_scale_inv as they are; A / sA as
 * for qx_gemm_fp8_blockscaled. Output as qx_silu_mul_quant's: Q (M x I)
 * e4m3 with leading dimension q_ld, Qs column-major (Qs[g * qs_ld + m]).
 * Bit-identical to qx_gemm_fp8_blockscaled of the same family followed by
 * qx_silu_mul_quant; the bf16 gate_up rows are never written. config: 10
 * (one workgroup per 256x256 tile) or 22 (persistent, as config 22 of
 * qx_gemm_fp8_blockscaled), the same bits as configs 10-22; 30 (the
 * promotion form, as config 30 of qx_gemm_fp8_blockscaled).
 */
int qx_gemm_fp8_swiglu_quant(const void* A, const float* sA, const void* W, const float* sW,
                             void* Q, int64_t q_ld, float* Qs, int64_t qs_ld, int64_t M,
                             int64_t I, int64_t K, int64_t lda, int64_t sa_ld, int config,
                             hipStream_t stream);

/*
 * Full-vocabulary log probabilities of t label tokens (t <= 16) for n rows:
 * out[r * out_ld + j] = bf16logit(r, targets[j]) - logsumexp_v bf16logit(r, v)
 * with bf16logit = bf16(normed[r] . head[v]) over all V head rows (bf16,
 * h_ld), in fp32 — the normalize=True path of AsyncLabelLogprobs.logprobs
 * (readout.py:164-200: F.linear over the whole head in blocks of rows,
 * logsumexp, the targets' columns). targets: int64 on the device, each in
 * [0, V). workspace: caller-allocated device memory of at least
 * qx_vocab_logprobs_workspace(n, V, t) bytes (per-block partial sums and
 * the target logits); H a multiple of 64.
 */
int64_t qx_vocab_logprobs_workspace(int64_t n, int64_t V, int64_t t);
int qx_vocab_logprobs(const void* normed, int64_t n_ld, const void* head, int64_t h_ld,
                      const int64_t* targets, int64_t t, float* out, int64_t out_ld, int64_t n,
                      int64_t V, int64_t H, void* workspace, int64_t workspace_bytes,
                      hipStream_t stream);

/*
 * qx_vocab_logprobs without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The same kernels, the same results bit for bit, over a workspace of the
 * library's own: one file-scope device array per GPU of
 * qx_vocab_logprobs_noalloc_max_bytes() bytes (8 MiB), held until the
 * process ends; its device address is looked up once per device with
 * hipGetSymbolAddress. Calls whose qx_vocab_logprobs_workspace(n, V, t)
 * exceeds it are rejected (-1 and a message). It allocates nothing and
 * needs nothing cleared (every workspace byte is written before it is
 * read). Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (several streams, several threads) race.
 */
int64_t qx_vocab_logprobs_noalloc_max_bytes(void);
int qx_vocab_logprobs_noalloc(const void* normed, int64_t n_ld, const void* head, int64_t h_ld,
                              const int64_t* targets, int64_t t, float* out, int64_t out_ld,
                              int64_t n, int64_t V, int64_t H, hipStream_t stream);

/*
 * Per-token 128-group e4m3 quant of bf16 rows. Replaces Engine.quant ->
 * vLLM per_token_group_quant_fp8 (attention.py:517-532).
 */
int qx_group_quant(const void* x, int64_t x_ld, void* q, int64_t q_ld, float* scales,
                   int64_t s_ld, int64_t n, int64_t K, hipStream_t stream);

/*
 * k_pool[dst[i]] = k[src[i]], v_pool[dst[i]] = v[src[i]] for rows of
 * row_elems 16-bit values; dst[i] < 0 writes nothing. Source rows have
 * strides k_ld and v_ld (v may be the strided v slice of qkv). K rows are
 * bf16 and copied; V rows are copied as they are, or with v_to_f16 the bf16
 * V rows go to an fp16 V pool (round to nearest even, saturated at
 * +-65504; the pool-to-pool tail copy runs without it). Replaces the Triton
 * kv_row_scatter
 * (attention.py:885-897) of Engine.kv_row_scatter / write_kv
 * (attention.py:1165-1195), including its pool-to-pool tail copy. With src
 * and dst both NULL, row i goes to row i (a contiguous copy, V converted:
 * the tree path's call A reads the pack's own rows that way).
 */
int qx_kv_scatter(const void* k, int64_t k_ld, const void* v, int64_t v_ld, void* k_pool,
                  void* v_pool, const int64_t* src, const int64_t* dst, int64_t count,
                  int64_t row_elems, int v_to_f16, hipStream_t stream);

/* out[i] = table[ids[i]] (bf16 rows). Replaces vLLM embed_tokens (qwen3.py:123). */
int qx_embed(const void* table, int64_t t_ld, const int64_t* ids, void* out, int64_t o_ld,
             int64_t n, int64_t H, hipStream_t stream);

/*
 * The most keys (used[s]) one sequence of a paged attention call may have:
 * 2560 pages of `page` tokens (40,960 at the arena's 16: Qwen3's whole
 * context), the page-table
 * row each workgroup stages in LDS. Host only; -1 (message in
 * qx_last_error()) for a page size the kernels do not take. No counterpart
 * in the reference (its paged kernel takes any block-table width); callers
 * refuse longer documents at admission (StageAdmission) rather than at the
 * first attention launch.
 */
int64_t qx_paged_attention_max_keys(int64_t page);

/*
 * Varlen GQA attention reading bf16 K and a bf16 (v_bf16 = 1, the
 * reference arena's pools) or fp16 (v_bf16 = 0) V pool through a block
 * table: sequence s has
 * query rows [cu_q[s], cu_q[s+1]) and keys [0, used[s]) at pool rows
 * table[s*table_ld + j/page]*page + j%page; causal masking aligned
 * bottom-right. Replaces Engine.attention_unified -> _paged ->
 * flash_attn_varlen_func(..., block_table, seqused_k, causal)
 * (attention.py:1477-1573, 1368-1393, 1280-1306); max_q and max_used are
 * FA's max_seqlen_q / max_seqlen_k (max_used <= 2048 * page). With out_fp8 it also
 * performs Engine.quant of the bf16 result (attention.py:1274-1275): e4m3
 * rows plus scales[h*s_ld + row] (one group per head, D == 128).
 * work/n_work: the work list (below) or NULL/0; tile_rows: the query rows
 * per workgroup it was built for (0: the default for (HQ / HK, D); 32 is
 * also accepted for D == 128 with HQ / HK a multiple of 4).
 */
int qx_paged_attention(const void* q, int64_t q_ld, const void* k_pool, const void* v_pool,
                       const int* cu_q, const int* used, const int* table, int64_t table_ld,
                       int64_t seqs, int64_t max_q, int64_t max_used, int64_t HQ, int64_t HK,
                       int64_t D, int64_t page, float scale, int causal, void* out_bf16,
                       void* out_fp8, int64_t o_ld, float* scales, int64_t s_ld,
                       const int* work, int64_t n_work, int64_t tile_rows, int v_bf16,
                       hipStream_t stream);

/*
 * qx_paged_attention (with the o_proj quant, D == 128) on q as the qkv
 * projection leaves it: q (the first HQ*128 columns of the qkv rows, q_ld
 * apart) is put through Qwen3's q-norm and neox RoPE per row as it is
 * loaded, with positions[i] (query row i), the (max_pos, 128) [cos | sin]
 * cache (fp32 with cs_is_f32, else bf16), the bf16 q-norm weight q_w and eps:
 * bit for bit what qx_qk_norm_rope_kv writes as q_out, whose pass then
 * writes K and V only (q_out NULL). Fuses the q half of Engine.qk_norm_rope
 * (attention.py:1251-1255 -> :833-879) into the attention call it feeds
 * (attention.py:1477-1573); saves q's write and re-read.
 */
int qx_paged_attention_qnorm(const void* q, int64_t q_ld, const void* k_pool, const void* v_pool,
                             const int* cu_q, const int* used, const int* table,
                             int64_t table_ld, int64_t seqs, int64_t max_q, int64_t max_used,
                             int64_t HQ, int64_t HK, int64_t D, int64_t page, float scale,
                             int causal, void* out_fp8, int64_t o_ld, float* scales, int64_t s_ld,
                             const int* work, int64_t n_work, int64_t tile_rows, int v_bf16,
                             const int64_t* positions, const void* cos_sin, int cs_is_f32,
                             const void* q_w, float eps, hipStream_t stream);

/*
 * Host function: the query rows per workgroup (work-list tile height) that a
 * paged call over these sequences runs best with: 32 where qx_paged_attention
 * accepts it and the default-height work items read at most 8 64-key tiles
 * on average (short documents: two 4-wave workgroups per CU hide each
 * other's fixed cost), else the default. cu_q and used are host copies.
 * Returns the rows or -1. No reference counterpart (FlashAttention's varlen
 * grid has one tile height).
 */
int64_t qx_paged_attention_tile_rows(const int* cu_q, const int* used, int64_t seqs, int64_t HQ,
                                     int64_t HK, int64_t D, int causal);

/*
 * Host function: the work list for qx_paged_attention's `work` argument
 * (device copy of it, n_work = the return value): one (sequence, query tile)
 * int pair per query tile of tile_rows rows (0: the default for (HQ / HK, D);
 * the call takes the same tile_rows) that holds rows, heaviest first (most
 * keys to read). With work == NULL the
 * call launches its full (max_q tiles x seqs) grid instead, whose tiles past
 * a sequence's rows exit at once. cu_q and used are host copies. Returns the
 * item count (<= capacity) or -1. No reference counterpart: FlashAttention's
 * varlen grid is the full one.
 */
int64_t qx_paged_attention_work(const int* cu_q, const int* used, int64_t seqs, int64_t HQ,
                                int64_t HK, int64_t D, int causal, int64_t tile_rows, int* work,
                                int64_t capacity);

/*
 * The tree attention path's two calls (Engine.attention_tree,
 * attention.py:1395-1441): each is flash_attn_varlen_func with
 * return_softmax_lse=True (attention.py:1280-1306). Writes bf16 out
 * (rows of o_ld elements, row i = query i in cu_q order) and
 * lse[h*lse_ld + i] = ln(sum_j exp(scale * q_i . k_j)) (-inf for a row that
 * sees no key).
 *   table != NULL, cu_k == NULL: call B, keys [0, used[s]) read through the
 *     block table as in qx_paged_attention (bf16 K pool, V as v_bf16 says);
 *   table == NULL, cu_k != NULL: call A, key j of sequence s is row
 *     cu_k[s] + j of k (bf16) and v (as v_bf16 says), rows of HK * D elements, and
 *     used[s] <= cu_k[s+1] - cu_k[s].
 * q_index (may be NULL): query i reads Q row q_index[i] (the reference's
 * q3.index_select(0, reads["rows"]), without the copy). causal aligns
 * bottom-right as in qx_paged_attention. work/n_work as there, built for the
 * default tile height (tile_rows 0).
 */
int qx_attention_lse(const void* q, int64_t q_ld, const int64_t* q_index, const void* k,
                     const void* v, const int* cu_q, const int* used, const int* table,
                     int64_t table_ld, const int* cu_k, int64_t seqs, int64_t max_q,
                     int64_t max_used, int64_t HQ, int64_t HK, int64_t D, float scale, int causal,
                     void* out_bf16, int64_t o_ld, float* lse, int64_t lse_ld, const int* work,
                     int64_t n_work, int v_bf16, hipStream_t stream);

/*
 * Replaces Engine.merge_attn_quant / the merge_attn_quant Triton kernel
 * (attention.py:902-948, QUANT on, UE8M0 off): for row t with
 * source[t] >= 0, w = bf16(sigmoid(lb[h*lb_ld + source[t]] - la[h*la_ld + t])),
 * y = bf16(a + (b[source[t]] - a) * w); otherwise y = a. Then per head
 * (D == 128, one 128-group) scale = max(amax|y|, 1e-10) / 448 and
 * e4m3(clamp(y / scale, +-448)) into q, scale into scales[h*s_ld + t].
 * With scales == NULL (QUANT off, any D in {64, 128}) the bf16 y goes to q.
 * q_ld is in elements of q; a, b, q rows hold HQ * D values.
 */
int qx_merge_attn_quant(const void* a, int64_t a_ld, const void* b, int64_t b_ld,
                        const float* la, int64_t la_ld, const float* lb, int64_t lb_ld,
                        const int* source, int64_t n, int64_t HQ, int64_t D, void* q,
                        int64_t q_ld, float* scales, int64_t s_ld, hipStream_t stream);

/*
 * Call C's merge into call B's output (merge_partial, attention.py:407-429,
 * called at :1424-1434 for label-path rows): for i < count and each head h,
 * with r = index[i], lb = lse[h*lse_ld + r], lc = lse_c[h*lse_c_ld + i],
 * top = max(lb, lc), wb = exp(lb - top), wc = exp(lc - top):
 * out[r, h] = bf16(out[r, h] * (wb / (wb + wc)) + out_c[i, h] * (wc / (wb + wc)))
 * and lse[h*lse_ld + r] = top + ln(wb + wc), in fp32. Rows hold H * D bf16
 * (o_ld, c_ld elements apart); index must not repeat. A (row, head) with no
 * keys on either side (top = -inf) is left unchanged.
 */
int qx_merge_partial(void* out, int64_t o_ld, float* lse, int64_t lse_ld, const int64_t* index,
                     const void* out_c, int64_t c_ld, const float* lse_c, int64_t lse_c_ld,
                     int64_t count, int64_t H, int64_t D, hipStream_t stream);

/*
 * Last-token answer head over the retained head rows (t <= 16):
 * logits = normed . rows^T; mode 0 rounds logits to bf16 (AnswerRows.logits,
 * AsyncLabelLogprobs normalize=False: readout.py:44-48, 188-191), mode 1
 * keeps fp32 (AsyncScores: readout.py:331-336). With cls (1 yes, 0 no,
 * -1 neither per row) it writes bits = max(yes) > max(no) (AI.IF),
 * yes_no pairs, and score = sigmoid((yes - no) / temperature) (AI.SCORE).
 * Any output pointer may be NULL.
 */
int qx_answer_head(const void* normed, int64_t n_ld, const void* rows, int64_t r_ld, int64_t t,
                   int64_t n, int64_t H, int mode, const int* cls, float temperature,
                   float* logits, uint8_t* bits, float* yes_no, float* score,
                   hipStream_t stream);

/*
 * Host function (no device work): the prefix tree of n documents, document i
 * being tokens[offsets[i] .. offsets[i+1]) (offsets[0] == 0, host memory).
 * order[k] = the k-th document in lexicographic token order (stable);
 * shared[i] = min(common prefix with its predecessor in that order,
 * len(i) - 1) rounded down to page_tokens; parent[i] = the document it
 * borrows from (its predecessor or, climbing, the nearest ancestor that
 * borrowed at least as much), -1 if shared[i] == 0. Replaces
 * PrefixIndex::new / PrefixIndex::tree (crates/quail-planner/src/inputs/
 * prefix.rs:33-73) behind PrefixTree (quail/common/tokens.py:440-484).
 */
int qx_prefix_tree(const int64_t* tokens, const int64_t* offsets, int64_t n,
                   int64_t page_tokens, int64_t* order, int64_t* parent, int64_t* shared);

/*
 * Host functions (no device work): page accounting of the paged KV arena.
 * Replace PageArena (quail/backends/quail/executor/pages.py:8-275), which
 * KVArena (arena.py:106-147,347-437,522-563) drives. A pool is an opaque
 * handle; keys are caller-chosen int64 ids (> 0; the packer's temporary
 * keys are < 0). Besides QX_OK / -1 (argument error), the calls return
 * -2 for a key that is not resident and -3 for one that already is.
 *
 * qx_pages_create: num_pages pages of page_tokens tokens; the free stack
 *   hands out 0, 1, 2, ... first (pages.py:26).
 * qx_pages_alloc (pages.py:63-81): pages for ceil(capacity / page) minus the
 *   borrowed ones; *allocated = their count, or -1 (nothing changed) when
 *   the free stack is short.
 * qx_pages_shared (pages.py:83-92): the parent's table pages holding its
 *   tokens [start, shared), both multiples of the page.
 * qx_pages_table: the key's table (borrowed, then owned pages) when cap
 *   holds it, and info = {tokens, borrowed, owned, pinned, retained,
 *   allocation order}.
 * qx_pages_stats: {free pages, retained pages, resident tokens, retained
 *   tokens, resident keys}.
 * qx_pages_keys: the resident keys in allocation order.
 * qx_pages_free_key / drop_leading / rewind / grow (pages.py:100-154):
 *   *out = pages freed (grow: pages added, or -1 when short).
 * qx_pages_pin / retain / pop_victim (pages.py:168-250): retained keys are
 *   evicted lowest priority first, ties in retention order; the default
 *   priority is tokens per page the key alone holds. victim = {found, key,
 *   pages it alone held, tokens}; the victim stays resident.
 * qx_pages_free_list: the free stack, bottom first.
 */
int qx_pages_create(int64_t num_pages, int64_t page_tokens, void** pool);
int qx_pages_destroy(void* pool);
int qx_pages_alloc(void* pool, int64_t key, int64_t tokens, int64_t capacity_tokens,
                   const int32_t* borrowed, int64_t n_borrowed, int64_t* allocated);
int qx_pages_shared(void* pool, int64_t parent, int64_t shared, int64_t start, int32_t* pages,
                    int64_t cap, int64_t* n);
int qx_pages_table(void* pool, int64_t key, int32_t* pages, int64_t cap, int64_t* info);
int qx_pages_stats(void* pool, int64_t* stats);
int qx_pages_keys(void* pool, int64_t* keys, int64_t cap, int64_t* n);
int qx_pages_free_key(void* pool, int64_t key, int64_t* freed);
int qx_pages_drop_leading(void* pool, int64_t key, int64_t pages, int64_t* freed);
int qx_pages_rewind(void* pool, int64_t key, int64_t tokens, int64_t* freed);
int qx_pages_grow(void* pool, int64_t key, int64_t capacity_tokens, int64_t* added);
int qx_pages_set_tokens(void* pool, int64_t key, int64_t tokens);
int qx_pages_pin(void* pool, int64_t key);
int qx_pages_retain(void* pool, int64_t key, int has_priority, double priority);
int qx_pages_pop_victim(void* pool, const int64_t* keep, int64_t n_keep, int64_t* victim);
int qx_pages_free_list(void* pool, int32_t* pages, int64_t cap, int64_t* n);

/*
 * Host function (no device work): one pack of the unified causal path.
 * Replaces pack_chunk with attention_mode="unified"
 * (quail/backends/quail/executor/chunk.py:505-1160; group loop :606-684,
 * unified pools :913-1054, _PoolBuilder :407-502). groups holds 8 int64 per
 * group: {key, fresh, f, start, prefix tokens, suffixes, suffix tokens kept
 * in the key's pages, every suffix row answers}; prefix_ids concatenates
 * the fresh groups' prefixes, suffix_lens and suffix_ids every group's
 * suffixes. A suffix that does not fit its key's pages gets a temporary key
 * (id < 0) in `pool`. On success *pack holds the arrays until
 * qx_pack_destroy; qx_pack_array(which) points at one of them:
 *   0 input ids, 1 positions, 2 final rows, 3 cu_a (int32), 4 rows per
 *   answer (empty unless some group answers on every row), 5 src, 6 dst,
 *   7 tail_src, 8 tail_dst, 9 cu_q (int32), 10 used (int32), 11 block table
 *   (int32, rows of `width`), 12 pages per sequence, 13 temporary keys,
 *   14 (row0, prefix end, row1) per group, 15 suffixes per group, 16 fresh
 *   keys, 17 {rows, max_q, max_used, multi-row, tail copies, width}.
 * On failure nothing stays allocated and *failed_group names the group;
 * -4 means the temporaries do not fit the free pages.
 */
int qx_pack_unified(void* pool, const int64_t* groups, int64_t n_groups,
                    const int64_t* prefix_ids, const int64_t* suffix_lens,
                    const int64_t* suffix_ids, void** pack, int64_t* failed_group);
int qx_pack_array(void* pack, int64_t which, const void** data, int64_t* count);
int qx_pack_destroy(void* pack);

#ifdef __cplusplus
}
#endif

#endif /* QUAIL_MI355X_H */
