/*
 * libmoc -- MI355X (gfx950) Mixture-of-Chapters memory cross-attention.
 *
 * C ABI: plain pointers, int64 sizes and a HIP stream.  Every pointer argument
 * is DEVICE memory unless stated otherwise.  Entry points never allocate,
 * never synchronise the host, and launch asynchronously on `stream`.  They
 * return MOC_OK (0) or an error code; moc_last_error() returns the message of
 * the last failure on the calling thread.  Shape/argument errors are reported
 * before anything is launched.
 *
 * Citations name the reference interface each entry point replaces
 * (paths relative to the Tasmay-Tibrewal/Memory repository root).
 *
 * Layouts used below:
 *   chapter-head tiles  K[u][hk][t][dh], V[u][hk][t][dh]   (u = de-duplicated chapter,
 *                        t < T tokens of the chapter, dh < Dh); every (u, hk) block is
 *                        contiguous.
 *   edge                 e = row * NS + slot of a (rows, NS) chapter-selection matrix.
 */
#ifndef MOC_H
#define MOC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

#define MOC_ABI_VERSION 1

/* status codes */
#define MOC_OK 0
#define MOC_ERR_ARG 1         /* bad pointer / shape / value (Python: ValueError) */
#define MOC_ERR_UNSUPPORTED 2 /* valid but not implemented for this shape/dtype  */
#define MOC_ERR_LAUNCH 3      /* HIP runtime error                               */

/* element types */
#define MOC_F32 0
#define MOC_BF16 1

/* row normalisation of gathered bank rows */
#define MOC_NORM_NONE 0
#define MOC_NORM_RMS 1
#define MOC_NORM_LAYERNORM 2

const char* moc_last_error(void);
int moc_abi_version(void);

/* ------------------------------------------------------------------ router */

/* Replaces the top-k block of ChapterRouter.forward (memory_transformer/router.py:114-149)
 * and of route_token_level (router.py:293-329): p = softmax(logits); when S > 0 the first S
 * chapters are zeroed and p renormalised; the k largest are selected (order: logit
 * descending, equal logits by ascending chapter id) and their weights renormalised.
 * logits f32 [R, C]; idx i32 [R, k] (global chapter ids); w f32 [R, k];
 * probs f32 [R, C] (optional, NULL to skip) receives softmax(logits).  k <= 1024. */
int moc_router_topk(const float* logits, int64_t R, int64_t C, int S, int k, int32_t* idx, float* w,
                    float* probs, hipStream_t stream);

/* Gradient of the chain above w.r.t. logits, given dw = dL/dw (f32 [R, k]).
 * Writes every element of dlogits f32 [R, C].  Same clamp_min(1e-12) gating as autograd. */
int moc_router_topk_bwd(const float* logits, const int32_t* idx, const float* dw, int64_t R, int64_t C, int S,
                        int k, float* dlogits, hipStream_t stream);
/* The per-token router's backward in one pass (router.py:294 + :114-149 autograd): the logit
 * gradient of moc_router_topk_bwd (plus dz_in f32 [R, C], the logits' own gradient from the
 * router losses, or NULL) is not stored; instead dzp bf16 [R, Cp] = its bf16 copy (columns
 * C .. Cp-1 zero; the operand of dx = dz W and dW = dz^T x on the chapter kernels) and the bias
 * gradient db f32 [C] = its column sums (fp32, fixed order; workspace from
 * moc_router_topk_bwd_pack_workspace).  R > 64, C <= Cp <= 4608, Cp even, k <= 64;
 * MOC_ERR_UNSUPPORTED outside that range (moc_router_topk_bwd + moc_logit_grad_pack then). */
size_t moc_router_topk_bwd_pack_workspace(int64_t R, int64_t C);
int moc_router_topk_bwd_pack(const float* logits, const int32_t* idx, const float* dw, int64_t R, int64_t C, int S,
                             int k, const float* dz_in, int64_t Cp, void* dzp, float* db, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

/* Replaces MemoryTransformer._prepend_shared_chapters (memory_transformer/model.py:356-391):
 * idx_star = [0..S-1, idx], omega = [1 (S times), scale * w] / sum.  S > 0.
 * idx i32 [R, k], w f32 [R, k] -> idx_star i32 [R, S+k], omega f32 [R, S+k]. */
int moc_prepend_shared(const int32_t* idx, const float* w, int64_t R, int k, int S, float scale, int32_t* idx_star,
                       float* omega, hipStream_t stream);
/* dw f32 [R, k] = d omega / d w applied to domega f32 [R, S+k] (overwrites dw). */
int moc_prepend_shared_bwd(const float* w, const float* domega, int64_t R, int k, int S, float scale, float* dw,
                           hipStream_t stream);

/* The sequence router's top-k followed by the shared-chapter prepend in one launch
 * (router.py:114-149 then model.py:356-391): idx / w as moc_router_topk, idx_star / omega as
 * moc_prepend_shared on them (bit-identical to the two separate calls).  S > 0. */
int moc_router_topk_prepend(const float* logits, int64_t R, int64_t C, int S, int k, float scale, int32_t* idx,
                            float* w, int32_t* idx_star, float* omega, hipStream_t stream);
/* Backward of that chain from the attention's d omega partials to the logits, one launch:
 * d omega[r, j] = sum_hk dom_part[(r (S+k) + j) HK + hk] (dom_part f32 [R (S+k), HK], as
 * moc_xattn_bwd_dkv writes it), then moc_prepend_shared_bwd and moc_router_topk_bwd (w = the
 * top-k's weights); dlogits f32 [R, C] also receives dz_in f32 [R, C] when non-NULL (a
 * gradient arriving at the logits from the router losses).  S <= 1024, C <= 8192. */
int moc_router_seq_bwd(const float* logits, const int32_t* idx, const float* w, const float* dom_part, int HK,
                       int64_t R, int64_t C, int S, int k, float scale, const float* dz_in, float* dlogits,
                       hipStream_t stream);

/* Replaces the pooling of ChapterRouter.forward (router.py:96-107 mean; :158-195 rolling
 * mean given as per-position coefficients coef f32 [L], NULL = mean).
 * h [B, L, d] of dtype; pooled f32 [B, d]; workspace from moc_router_pool_workspace. */
size_t moc_router_pool_workspace(int64_t B, int64_t L, int64_t d);
int moc_router_pool(const void* h, int dtype, int64_t B, int64_t L, int64_t d, const float* coef, float* pooled,
                    void* workspace, size_t workspace_bytes, hipStream_t stream);
/* The same pooling in one launch, without a workspace, for d % 8 == 0 and 16-byte aligned h. */
int moc_router_pool1(const void* h, int dtype, int64_t B, int64_t L, int64_t d, const float* coef, float* pooled,
                     hipStream_t stream);
/* Backward of the pooling added into an existing gradient (autograd's accumulation of the two
 * uses of hidden_states, router.py:96-107 and the q projection): x [B, L, d] of dtype +=
 * v f32 [B, d] * (coef ? coef[l] : scale), in place.  d % 8 == 0, 16-byte aligned. */
int moc_rows_add_bcast(void* x, int dtype, int64_t B, int64_t L, int64_t d, const float* v, const float* coef,
                       float scale, hipStream_t stream);

/* Replaces ChapterRouter.router (nn.Linear(d, C, bias=True), router.py:64) for few rows:
 * logits f32 [R, C] = x f32 [R, d] . W[C, d]^T + bias f32 [C] (bias may be NULL). */
int moc_router_linear(const float* x, int64_t R, int64_t d, const void* W, int w_dtype, const float* bias, int64_t C,
                      float* logits, hipStream_t stream);
/* Backward of moc_router_linear: dx f32 [R, d], dW f32 [C, d], db f32 [C]; any may be NULL. */
size_t moc_router_linear_bwd_workspace(int64_t R, int64_t d, int64_t C);
int moc_router_linear_bwd(const float* dz, const float* x, int64_t R, int64_t d, const void* W, int w_dtype,
                          int64_t C, float* dx, float* dW, float* db, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* The per-token router's logit gradient dz f32 [R, C] as the bf16 operand of its backward
 * products (the input and weight gradients of ``self.router(hidden_states)``, router.py:294):
 * dzp bf16 [R, Cp] (row stride Cp, even, >= C; columns C .. Cp-1 zero), and when db != NULL the
 * bias gradient db f32 [C] = sum over rows of dz (fp32, fixed order; workspace from
 * moc_logit_grad_pack_workspace).  One read of dz. */
size_t moc_logit_grad_pack_workspace(int64_t R, int64_t C);
int moc_logit_grad_pack(const float* dz, int64_t R, int64_t C, int64_t Cp, void* dzp, float* db, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* Replaces ChapterRouter._compute_losses (router.py:197-260) for rows of logits f32 [R, C] and
 * the selected chapter ids idx i32 [R, k] (entries outside [0, C) are ignored):
 * losses f32 [4] = {load_balance, auxiliary, z_loss, entropy} with p = softmax(logits) per row,
 *   load_balance = C sum_c f_c P_c (f_c = selections of c / R, P_c = mean_r p_rc),
 *   auxiliary = mean_c (mean_r p_rc^2 - 1/C)^2, z_loss = mean_r lse_r^2,
 *   entropy = -mean_r sum_c p_rc log(max(p_rc, 1e-12)).
 * Also writes counts i32 [C] (selections per chapter) and what the backward reads: row_lse
 * f32 [R] and col_coef f32 [C][2] (8-byte aligned) = {C counts_c / R^2,
 * 4 (mean_r p_rc^2 - 1/C) / (C R)}.  Deterministic (fixed-order sums, integer counts).
 * C <= 16384. */
size_t moc_router_losses_workspace(int64_t R, int64_t C);
int moc_router_losses(const float* logits, int64_t R, int64_t C, const int32_t* idx, int k, float* row_lse,
                      float* col_coef, int32_t* counts, float* losses, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);
/* dlogits f32 [R, C] = d(sum_i dlosses[i] losses[i]) / d logits, dlosses f32 [4] on the device
 * (the selection counts are constants, as the reference's one-hot is). */
int moc_router_losses_bwd(const float* logits, int64_t R, int64_t C, const float* row_lse, const float* col_coef,
                          const float* dlosses, float* dlogits, hipStream_t stream);

/* ------------------------------------------------------------- chapter plan */

/* De-duplicates the chapters of E edges and builds the chapter -> edges inverted index
 * (a stable counting sort; the reference builds it with argsort + searchsorted,
 * kernels-final/kernel_v4.py:213-257).  chap i32 [E] in [0, C) (others are skipped).
 * uniq i32 [min(E, C)], n_uniq i32 [2] = {distinct chapters, skipped edges},
 * edge_u i32 [E] (-1 for skipped), csr_off i32 [min(E, C) + 1], csr_edge i32 [E].
 * C <= 16384. */
size_t moc_chapter_plan_workspace(int64_t E, int64_t C);
int moc_chapter_plan(const int32_t* chap, int64_t E, int64_t C, void* workspace, size_t workspace_bytes,
                     int32_t* uniq, int32_t* n_uniq, int32_t* edge_u, int32_t* csr_off, int32_t* csr_edge,
                     hipStream_t stream);
/* moc_chapter_plan without a caller workspace and without allocating: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  The workspace is a fixed 4 MiB device array
 * of the library (one per GPU, held until the process ends), so E and C are limited to
 * moc_chapter_plan_workspace(E, C) <= 4 MiB (e.g. E <= 258,048 edges over 4,097 chapters);
 * larger plans return MOC_ERR_UNSUPPORTED.  Every call on a GPU shares that array: calls that
 * overlap on one GPU (concurrent streams) race and must not be issued.  The first call on each
 * device looks the array's device address up (hipGetSymbolAddress): make it outside stream
 * capture; later calls only launch kernels (no memset, no allocation) and may be captured into a
 * HIP graph and replayed. */
int moc_chapter_plan_noalloc(const int32_t* chap, int64_t E, int64_t C, int32_t* uniq, int32_t* n_uniq,
                             int32_t* edge_u, int32_t* csr_off, int32_t* csr_edge, hipStream_t stream);

/* --------------------------------------------------- gather + K/V projection */

/* Per-row statistics of the gathered rows for MemoryTransformer._normalize_shared_routed_memory_vectors
 * (memory_transformer/model.py:393-432): mean f32 and rstd f32 [max_u * T]. */
int moc_row_stats(const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq, const int32_t* n_uniq,
                  int64_t max_u, int norm, float eps, float* mean, float* rstd, hipStream_t stream);

/* Replaces ChapteredMemoryBank.get_chapters_batched (memory_transformer/memory_bank.py:244-293)
 * followed by k_proj/v_proj of MemoryCrossAttention._compute_qkv (memory_attention.py:241-243),
 * computed once per distinct chapter.  bank [N_m, d] (bf16 or f32), wkv [2*HK*Dh, d] of dtype
 * (= [Wk; Wv]); row_mean/row_rstd from moc_row_stats or both NULL.  Outputs (each may be NULL,
 * but K and V each need one form): chapter-head tiles k_tiles, v_tiles [max_u][HK][T][Dh] (the
 * form every attention entry point here reads) and, optionally, their transposes kt_tiles,
 * vt_tiles [max_u][HK][Dh][T], of dtype.  The key axis of the
 * transposed tiles is stored in MFMA key order: within each 32-key group, key 4g + e sits at
 * position 8g + e and key 16 + 4g + e at 8g + 4 + e (g, e < 4).  d % 64 == 0,
 * (2*HK*Dh) % 128 == 0, T % 32 == 0 when a transposed output is requested. */
int moc_kv_project(int dtype, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                   const int32_t* n_uniq, int64_t max_u, const float* row_mean, const float* row_rstd,
                   const void* wkv, int HK, int Dh, void* k_tiles, void* v_tiles, void* kt_tiles, void* vt_tiles,
                   hipStream_t stream);

/* K/V projection of the plan's distinct chapters on the matrix cores, the gather fused into the
 * operand loads: y[c*64 + j][n] = sum_k X_c[j][k] * w[n][k] for c < n_uniq, j < 64, where
 * X_c is bank rows uniq[c]*64 .. +63 (gather != 0; rows = the bank) or rows c*64 .. +63 of a
 * contiguous block (gather == 0; e.g. moc_gather_rows output).  rows bf16 with row stride ld
 * elements, w [N][K] bf16 (= [Wk; Wv], N = 2*HK*Dh), y [max_u*64][ldy] bf16; rows of plan slots
 * >= n_uniq are not written.  Replaces ChapteredMemoryBank.get_chapters_batched
 * (memory_transformer/memory_bank.py:263-293) followed by k_proj / v_proj of
 * MemoryCrossAttention._compute_qkv (memory_attention.py:241-243), once per distinct chapter;
 * the result is the "projection rows" K / V layout of moc_xattn_fwd.  N % 256 == 0,
 * K % 64 == 0, T == 64. */
int moc_chapter_project(const void* rows, int64_t ld, int gather, const int32_t* uniq, const int32_t* n_uniq,
                        int64_t max_u, const void* w, int N, int K, void* y, int64_t ldy, hipStream_t stream);
/* Input gradient of that projection summed over each chapter's edges and stored per chapter:
 * out_c = (sum over the chapter's edges e, csr order, of dkv_edge rows e*64 .. +63) w_t^T, i.e.
 * out_c[j][n] = sum_k dK|dV_c[j][k] * w_t[n][k] with w_t [N = d][K = 2*HK*Dh] = [Wk; Wv]^T
 * (moc_weight_pack).  dkv_edge [E*64][ld] bf16 from moc_xattn_bwd_dkv; chapters with several
 * edges are read from red [max_u*64][ld] bf16, their sums from moc_dkv_multi_reduce.
 * out_bank_rows != 0: out is the dense bank gradient [N_m][ldo] and chapter c's rows are stored
 * at uniq[c]*64 .. +63 (the scatter-add of the gather's backward, memory_bank.py:287-291:
 * distinct chapters own distinct rows, so they are stored; the rest must be zero already);
 * out_bank_rows == 0: out [max_u*64][ldo], chapter c at rows c*64 .. (for a normalised bank or
 * a row-sparse gradient, finished by moc_bank_scatter / moc_bank_grad_accumulate without csr).
 * out_dtype MOC_BF16 or MOC_F32.  Replaces the autograd input gradient of k_proj / v_proj
 * (memory_attention.py:241-243) through get_chapters_batched (memory_bank.py:263-293). */
int moc_chapter_dx(const void* dkv_edge, int64_t ld, const int32_t* uniq, const int32_t* n_uniq, int64_t max_u,
                   const int32_t* csr_off, const int32_t* csr_edge, void* red, const void* w_t, int N, int K,
                   int out_dtype, void* out, int64_t ldo, int out_bank_rows, hipStream_t stream);
/* y [R][N] = x [R][K] w^T on the chapter GEMM (bf16 in and out, fp32 accumulation), x and y row
 * strides ldx, ldy: the bias-free nn.Linear of the memory layer's q_proj / o_proj
 * (memory_transformer/memory_attention.py:140-143, :241, :456) and its input gradient (w = the
 * transposed weight).  N % 256 == 0, K % 64 == 0. */
int moc_rows_linear(const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, void* y, int64_t ldy,
                    hipStream_t stream);
/* y [R][N] = res [R][N] + x [R][K] w^T in one GEMM (bf16 in and out, the residual added to the
 * fp32 product before the one rounding): the memory sublayer's o_proj with its residual add,
 * memory_transformer/memory_block.py:549-558 (``hidden_states = residual + mem_output`` after
 * memory_attention.py:456 ``self.o_proj(attn_output)``).  res row stride ldr (a multiple of 8,
 * 16-byte aligned); res may equal y (each element is read before it is written, by the same
 * lane).  N % 256 == 0, K % 64 == 0. */
int moc_rows_linear_residual(const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, const void* res,
                             int64_t ldr, void* y, int64_t ldy, hipStream_t stream);
/* y [R][N] f32 = x [R][K] w^T (+ bias [N] f32 when bias != NULL) for any N (w [N][K] bf16, K % 64
 * == 0; y row stride ldy >= N, any value): the per-token router logits, ``self.router(hidden)``
 * of ChapterRouter.route_token_level (memory_transformer/router.py:294), with operands in bf16
 * and the logits accumulated and kept in fp32. */
int moc_rows_linear_f32(const void* x, int64_t ldx, int64_t R, const void* w, int N, int K, const float* bias,
                        float* y, int64_t ldy, hipStream_t stream);
/* The memory sublayer's memory_layernorm folded into its q projection (memory_block.py:549-558:
 * q_proj(memory_layernorm(hidden)); RMSNorm memory_block.py:18-28 or nn.LayerNorm): y = norm(x) W^T
 * for x [R, K] bf16 (row stride ldx) without writing the normalised rows.  moc_norm_fold_weight
 * takes W [N, K] bf16, gamma f32 [K] and (LayerNorm) beta f32 [K] or NULL and writes
 * w_out = W diag(gamma) bf16 [N, K], u f32 [N] = row sums of w_out and v f32 [N] = W beta (u and v
 * for LayerNorm only; NULL for RMSNorm; beta NULL = no bias, v = 0).  moc_rows_linear_norm (norm
 * MOC_NORM_RMS or MOC_NORM_LAYERNORM) then computes y [R, N] bf16 = rstd (x w_out^T) (RMSNorm) or
 * rstd (x w_out^T - mean u) + v (LayerNorm), the row statistics over the K columns of x (fp32
 * sums; rstd = 1 / sqrt(mean(x^2) or var + eps)) taken inside the GEMM and written to rstd_out /
 * mean_out [R] f32 when non-NULL (what moc_row_norm_bwd reads).  N a multiple of 256, K of 64. */
int moc_norm_fold_weight(const void* w, int N, int K, const float* gamma, const float* beta, void* w_out, float* u,
                         float* v, hipStream_t stream);
int moc_rows_linear_norm(const void* x, int64_t ldx, int64_t R, const void* w_folded, int N, int K, int norm,
                         float eps, const float* u, const float* v, void* y, int64_t ldy, float* mean_out,
                         float* rstd_out, hipStream_t stream);
/* Sums of the per-edge dK|dV rows of the chapters selected by more than one edge (csr order,
 * fp32 accumulation, rounded to bf16): red [max_u*64][ld] (rows of other chapters untouched).
 * Feeds moc_chapter_dx and moc_chapter_wgrad, which read a single-edge chapter's rows in place
 * (the reference accumulates per chapter with its inverted-index kernel,
 * kernels-final/kernel_v4.py:534-671). */
int moc_dkv_multi_reduce(const void* dkv_edge, int64_t ld, const int32_t* n_uniq, int64_t max_u,
                         const int32_t* csr_off, const int32_t* csr_edge, void* red, hipStream_t stream);
/* Weight gradient of the K/V projection from the per-chapter rows: dw [N][K] (out_dtype f32 or
 * bf16) = sum over chapters c < n_uniq of dK|dV_c^T X_c, with dK|dV_c read like moc_chapter_dx
 * (one edge in place, several from red) and X_c the chapter's bank rows uniq[c]*64 .. (gather
 * != 0, x = the bf16 bank, row stride ldx) or rows c*64 .. of a contiguous bf16 block (gather
 * == 0, e.g. moc_gather_rows output for a normalised bank).  Replaces the autograd weight
 * gradient of k_proj / v_proj (memory_transformer/memory_attention.py:241-243) over the gathered
 * rows (memory_bank.py:263-293).  The chapters are split over several workgroups per 256 x 256
 * output tile; ws (moc_chapter_wgrad_workspace bytes) holds their fp32 partials, summed in a
 * fixed order.  N, K multiples of 256. */
size_t moc_chapter_wgrad_workspace(int N, int K, int64_t max_u);
int moc_chapter_wgrad(const void* dkv_edge, int64_t lda, const void* red, const void* x, int64_t ldx, int gather,
                      const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                      const int32_t* csr_edge, int N, int K, void* ws, size_t ws_bytes, int out_dtype, void* dw,
                      hipStream_t stream);
/* wkv [2*kv][d] bf16 = [wk; wv] and / or wkv_t [d][2*kv] bf16 = its transpose (either may be
 * NULL), from wk, wv [kv][d] of MOC_F32 / MOC_BF16: the concatenated K/V weight that the
 * chapter GEMMs read (the reference keeps k_proj and v_proj as two nn.Linear,
 * memory_transformer/memory_attention.py:140-143). */
int moc_weight_pack(const void* wk, int wk_dtype, const void* wv, int wv_dtype, int64_t kv, int64_t d, void* wkv,
                    void* wkv_t, hipStream_t stream);
/* wt [K][ldt] bf16 = w^T for w [N][K] of MOC_F32 / MOC_BF16, columns N .. ldt-1 zero: the
 * transposed (and zero-padded) weight operand of an input-gradient product on the rows GEMM,
 * e.g. dx = dlogits W of the per-token router (router.py:294) with its chapter count padded to a
 * multiple of 256.  K and ldt multiples of 8, ldt >= N; 16-byte aligned w and wt. */
int moc_weight_transpose(const void* w, int w_dtype, int64_t N, int64_t K, void* wt, int64_t ldt,
                         hipStream_t stream);

/* ------------------------------------------- the whole sequence-routed layer */

/* One memory layer of MemoryTransformer.forward with sequence-level routing and its sublayer
 * call (memory_transformer/model.py:609-692, memory_block.py:549-558 without the caller's norm
 * and residual; router.py:96-149, model.py:356-391, memory_attention.py:241-243, :269-478) as
 * one host call per direction: the library's router, chapter-plan, chapter-GEMM, attention and
 * weight-gradient entry points ordered over the caller's stream `main` and the side streams
 * `aux` (and `fill` in the backward), joined back into `main` by events before returning.
 * Shapes: h [B, L, d] bf16, d = 64 H (head_dim 64), d and 2*HK*64 multiples of 256, T = 64,
 * bank [N_m, d] bf16 (plain rows: no row norm), wr [C, d] f32 or bf16 (wr_dtype), br f32 [C] or
 * NULL, wq / wo [d, d], wk / wv [HK*64, d] bf16, coef f32 [L] (rolling-mean pooling) or NULL
 * (mean), 1 <= S <= 1024 shared chapters, 1 <= k <= min(1024, C - S), C <= 8192, B <= 64.
 * forward outputs: out [B, L, d] bf16 (after o_proj), logits f32 [B, C], idx i32 [B, k] (routed
 * global ids), idx_star i32 [B, S+k] and omega f32 [B, S+k] (after the prepend); `saved`
 * (moc_seq_layer_saved_bytes) holds what the backward reads and must reach it unchanged.
 * backward: dout [B, L, d] bf16, dlogits f32 [B, C] or NULL (a gradient at the logits from the
 * router losses); outputs, each NULL when not wanted: dh [B, L, d] bf16, dbank [bank_rows, d]
 * bf16 (dense: zeros except the selected chapters' rows), dwr f32 [C, d], dbr f32 [C], dwq and
 * dwo [d, d] bf16, dwkv [2*HK*64, d] (= [dWk; dWv], dwkv_dtype f32 or bf16); `scratch`
 * (moc_seq_layer_scratch_bytes) is working memory.  Both return 0 sizes for unsupported shapes.
 * Calls on one device must be issued from one host thread at a time. */
size_t moc_seq_layer_saved_bytes(int64_t B, int64_t L, int64_t d, int H, int HK, int64_t C, int S, int k);
size_t moc_seq_layer_scratch_bytes(int64_t B, int64_t L, int64_t d, int H, int HK, int64_t C, int S, int k);
int moc_seq_layer_fwd(const void* h, const void* bank, const void* wr, int wr_dtype, const float* br, const void* wq,
                      const void* wk, const void* wv, const void* wo, const float* coef, int64_t B, int64_t L,
                      int64_t d, int H, int HK, int64_t C, int S, int k, float routed_scale, void* out,
                      float* logits, int32_t* idx, int32_t* idx_star, float* omega, void* saved, size_t saved_bytes,
                      hipStream_t main, hipStream_t aux);
int moc_seq_layer_bwd(const void* h, const void* bank, const void* wr, int wr_dtype, const float* coef, int64_t B,
                      int64_t L, int64_t d, int H, int HK, int64_t C, int S, int k, float routed_scale,
                      const float* logits, const int32_t* idx, const float* omega, const void* saved,
                      size_t saved_bytes, const void* dout, const float* dlogits, void* dh, void* dbank,
                      int64_t bank_rows, float* dwr, float* dbr, void* dwq, void* dwkv, int dwkv_dtype, void* dwo,
                      void* scratch, size_t scratch_bytes, hipStream_t main, hipStream_t aux, hipStream_t fill);
/* Stage timing of the two calls above (no counterpart in the reference, which times whole steps
 * with torch.cuda.Event in its benchmarks, kernels-final/benchmark_kernels_final.py): stage s is
 * one or a few launches on one stream, named by moc_seq_layer_stage_name(s) (the entry point
 * and, where it is called more than once, its role).  moc_seq_layer_timing(mask, capacity) arms
 * the stages whose bit is set in `mask` on the current device (timing events around each of
 * their next `capacity` launches, on the stage's own stream; mask 0 disarms) and clears the
 * counts; moc_seq_layer_timing_read waits for the recorded events and returns, per stage, the
 * summed milliseconds, the timed launches and the launches past `capacity` (dropped may be
 * NULL), then clears the counts.  Not for use under graph capture. */
int moc_seq_layer_stage_count(void);
const char* moc_seq_layer_stage_name(int stage);
int moc_seq_layer_timing(uint64_t stage_mask, int capacity);
int moc_seq_layer_timing_read(double* total_ms, int32_t* launches, int32_t* dropped, int n);

/* ------------------------------------------------- routed attention forward */

/* Replaces MemoryCrossAttention._attention on omega-weighted gathered memory
 * (memory_transformer/model.py:689-692 + memory_attention.py:458-478, :269-318) for the
 * sequence-level path: one joint softmax over the NS selected chapters of each sequence,
 * with omega scaling both logits and values.  q [B, L, H, Dh].  K / V of the plan's chapters:
 * element (t, dh) of (chapter slot u, kv head hk) at k + u*su + hk*sh + t*st + dh (and the same
 * offsets from v), each base readable for kv_span elements (< 4 GiB; strides in elements,
 * 16-byte multiples, st >= 64): the chapter-head tiles of moc_kv_project are (HK*T*Dh, T*Dh, Dh);
 * projection rows [max_u*T][2*HK*Dh] (K columns, then V) are (T*2*HK*Dh, Dh, 2*HK*Dh) with
 * v = k + HK*Dh.  slot_u i32 [B, NS] (the plan's edge_u); omega f32 [B, NS]; out [B, L, H, Dh];
 * lse f32 [B, H, round_up(L, 128)] (log2 domain, +inf in the padding; consumed by the backward).
 * Dh == 64, T == 64. */
int moc_xattn_fwd(int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span, int64_t su,
                  int sh, int st, const int32_t* slot_u, const float* omega, int64_t B, int64_t L, int H, int HK, int Dh, int T,
                  int NS, float scale, void* out, float* lse, hipStream_t stream);
/* The attention weights of that forward (MemoryCrossAttention.forward with return_attn_weights,
 * memory_transformer/memory_attention.py:437-447: softmax(q k^T * scale) over each sequence's
 * NS * T selected, omega-weighted keys): weights [B, H, L, NS * T] (dtype), column c * T + j for
 * key j of slot c, from q, the K of moc_xattn_fwd's layout and the lse it wrote; skipped slots
 * (slot_u < 0) get 0.  q, k_tiles and weights 16-byte aligned. */
int moc_xattn_weights(int dtype, const void* q, const void* k_tiles, int64_t kv_span, int64_t su, int sh, int st,
                      const int32_t* slot_u, const float* omega, int64_t B, int64_t L, int H, int HK, int Dh, int T,
                      int NS, float scale, const float* lse, void* weights, hipStream_t stream);

/* ------------------------------------------------ routed attention backward */

/* Backward of moc_xattn_fwd (autograd of memory_transformer/memory_attention.py:301-316 through
 * the omega weighting of model.py:689-692).  Rows of lse / delta / qt / dot have stride
 * Lp = round_up(L, 128) (moc_xattn_fwd writes lse that way, padded with +inf).
 * prep: delta f32 [B, H, Lp] = rowsum(dout * out); optionally (both non-NULL) qt, dot
 * [B, H, Dh, Lp] (dtype) = q and dout transposed per (sequence, head), zero-padded, query axis
 * in MFMA key order (no entry point here needs them: moc_xattn_bwd_dkv reads q / dout). */
int moc_xattn_bwd_prep(int dtype, const void* q, const void* out, const void* dout, int64_t B, int64_t L, int H,
                       int Dh, float* delta, void* qt, void* dot, hipStream_t stream);
/* dq [B, L, H, Dh] (dtype); K / V as for moc_xattn_fwd. */
int moc_xattn_bwd_dq(int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span,
                     int64_t su, int sh, int st, const int32_t* slot_u, const float* omega, const void* dout, const float* lse,
                     const float* delta, int64_t B, int64_t L, int H, int HK, int Dh, int T, int NS, float scale,
                     void* dq, hipStream_t stream);
/* moc_xattn_bwd_dq with the prep's delta fused in: out [B, L, H, Dh] (dtype) is the forward's
 * output; delta f32 [B, H, Lp] = rowsum(dout * out) is written (padded rows 0) for
 * moc_xattn_bwd_dkv, from the dout rows the dq kernel reads anyway, so moc_xattn_bwd_prep is not
 * needed.  Same reference interface as prep + dq (the FlashAttention-style backward pre-pass and dQ
 * of memory_transformer/memory_attention.py:301-316's autograd). */
int moc_xattn_bwd_dq_delta(int dtype, const void* q, const void* k_tiles, const void* v_tiles, int64_t kv_span,
                           int64_t su, int sh, int st, const int32_t* slot_u, const float* omega, const void* out,
                           const void* dout, const float* lse, float* delta, int64_t B, int64_t L, int H, int HK, int Dh,
                           int T, int NS, float scale, void* dq, hipStream_t stream);
/* dK/dV per edge (edge e = b * NS + slot): dkv_edge [B * NS * T][2 * HK * Dh] (dtype) holds for
 * the chapter in slot `slot` of sequence b the rows [dL/dk (all kv heads) | dL/dv], where
 * dL/dk, dL/dv are gradients w.r.t. the unweighted projected keys/values (omega folded in).
 * Rows of skipped slots are not written.  domega_part f32 [B * NS][HK]: per (edge, kv head)
 * parts of dL/domega (caller sums over HK; skipped edges get 0). */
int moc_xattn_bwd_dkv(int dtype, const void* q, const void* dout,
                      const void* k_tiles, const void* v_tiles, int64_t kv_span, int64_t su, int sh, int st,
                      const int32_t* slot_u, const float* omega,
                      const float* lse, const float* delta, int64_t B, int64_t L, int H, int HK, int Dh, int T,
                      int NS, float scale, void* dkv_edge, float* domega_part, hipStream_t stream);
/* Sums the per-edge rows per distinct chapter following the plan's inverted index (the
 * reference accumulates per chapter with its inverted-index kernel,
 * kernels-final/kernel_v4.py:534-671): dkv [max_u * 64][row_elems] (dtype); rows of unused
 * plan slots are written as zero.  Fixed summation order (deterministic). */
int moc_dkv_reduce(int dtype, const void* dkv_edge, const int32_t* n_uniq, const int32_t* csr_off,
                   const int32_t* csr_edge, int64_t max_u, int64_t row_elems, void* dkv, hipStream_t stream);

/* Weight gradient of the K/V projection with the chapter gather (and row norm) fused:
 * dw [KV2][d] (out_dtype f32 or bf16) = dkv^T X, X[r] = norm(bank[uniq[r / 64] * 64 + r % 64]),
 * over the plan's n_uniq * 64 rows; dkv [max_u * 64][KV2] bf16 from moc_dkv_reduce.  With edge_u
 * (the plan's edge -> distinct chapter map) dkv is instead the per-edge rows of moc_xattn_bwd_dkv
 * ([E * 64][KV2], max_u = E): edge e's rows pair with the rows of chapter uniq[edge_u[e]], and
 * skipped edges (edge_u < 0) contribute nothing, so no per-chapter reduction is needed.  Replaces the
 * autograd weight gradient of k_proj / v_proj (memory_transformer/memory_attention.py:241-243)
 * over the gathered rows (memory_transformer/memory_bank.py:263-293).  T must be 64.  The rows
 * are split over several workgroups per output tile; ws (moc_kv_wgrad_workspace bytes) holds
 * their fp32 partials, summed in a fixed order. */
size_t moc_kv_wgrad_workspace(int64_t KV2, int64_t d, int64_t max_u);
int moc_kv_wgrad(const void* dkv, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                 const int32_t* n_uniq, const int32_t* edge_u, int64_t max_u, const float* row_mean,
                 const float* row_rstd, int64_t KV2, void* ws, size_t ws_bytes, int out_dtype, void* dw,
                 hipStream_t stream);
/* Same kernel over dense rows: dw [N][K] (out_dtype) = dy^T x with dy [R][N] bf16 and x [R][K]
 * (x_dtype bf16 or f32, rounded to bf16 for the MFMA).  The weight gradient of the memory
 * layer's bias-free q_proj / o_proj (memory_transformer/memory_attention.py:140-143, :241, :456),
 * which the reference gets from autograd of nn.Linear; R is the token count. */
size_t moc_linear_wgrad_workspace(int64_t R, int64_t N, int64_t K);
int moc_linear_wgrad(const void* dy, const void* x, int x_dtype, int64_t R, int64_t N, int64_t K, void* ws,
                     size_t ws_bytes, int out_dtype, void* dw, hipStream_t stream);
/* Gathered (and normalised) rows X [max_u * T][d] in dtype for the weight-gradient GEMM
 * dWkv = dkv^T X; rows of unused plan slots are zero. */
int moc_gather_rows(int dtype, const void* bank, int bank_dtype, int64_t d, int T, const int32_t* uniq,
                    const int32_t* n_uniq, int64_t max_u, const float* row_mean, const float* row_rstd, void* out,
                    hipStream_t stream);

/* Backward of the gather (memory_bank.py:287-291, a scatter-add into the bank gradient) through
 * the optional row normalisation: grad_bank[uniq[u]*T + t, :] = norm_bwd(g), g = dX[u*T + t, :]
 * (dX [max_u * T][d], one row per distinct-chapter row) or, when the plan's csr_off / csr_edge are
 * given, g = sum over the chapter's edges e (csr order) of dX[e*T + t, :] (dX [E * T][d], one row
 * per edge row).  Distinct chapters own distinct rows, so the rows are stored, not added;
 * grad_bank must be zero elsewhere.  dX of dx_dtype, grad_bank of bank_dtype. */
int moc_bank_scatter(int dx_dtype, const void* dX, const void* bank, int bank_dtype, int64_t d, int T,
                     const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                     const int32_t* csr_edge, const float* row_mean, const float* row_rstd, int norm,
                     void* grad_bank, hipStream_t stream);

/* Zero fill of `bytes` (multiple of 16, 16-byte aligned address) by `workgroups` one-wave
 * workgroups: the zeros of the dense bank gradient (autograd's zero-initialised result of the
 * gather, memory_bank.py:287-291, before moc_bank_scatter stores the selected rows), sized to
 * run beside the attention backward on a second stream rather than as a full-chip fill. */
int moc_fill_zero(void* dst, int64_t bytes, int workgroups, hipStream_t stream);

/* Row-sparse bank gradient (no counterpart in the reference, whose bank gradient is the dense
 * autograd result of the gather, memory_bank.py:287-291): the same rows as moc_bank_scatter,
 * accumulated in f32 grad_acc [N_m][d] for the chapters of the current `epoch`.  chap_epoch
 * i32 [C] tags which chapters already hold rows for the epoch: a chapter's first contribution
 * is stored, later ones (other layers sharing the bank, further micro-batches) are added, so
 * the accumulator is never zero-filled.  fresh i32 [max_u] is scratch. */
int moc_bank_grad_accumulate(int dx_dtype, const void* dX, const void* bank, int bank_dtype, int64_t d, int T,
                             const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, const int32_t* csr_off,
                             const int32_t* csr_edge, const float* row_mean, const float* row_rstd, int norm,
                             int epoch, int32_t* chap_epoch, int32_t* fresh, float* grad_acc, hipStream_t stream);

/* ------------------------------------------------------------ few-row linear */

/* y [M][N] = x [M][K] W[N][K]^T for M <= 256 rows (bf16 x and W, fp32 accumulation, y bf16 or
 * f32): the decode step's q_proj / o_proj (memory_attention.py:140-143, :241, :456) on one
 * token per sequence.  K % 128 == 0, N % 16 == 0, 16-byte aligned x and W. */
int moc_linear_rows(const void* x, int64_t M, int64_t K, const void* W, int64_t N, int out_dtype, void* y,
                    hipStream_t stream);

/* ------------------------------------------------------- caller-side norm */

/* The memory sublayer's `memory_layernorm` (memory_transformer/memory_block.py:549-558):
 * norm MOC_NORM_RMS = RMSNorm (memory_block.py:18-28, y = x / sqrt(mean(x^2) + eps) * w) or
 * MOC_NORM_LAYERNORM (nn.LayerNorm, y = (x - mu) / sqrt(var + eps) * w + b) over rows x [R][d]
 * (d % 8 == 0, d <= 2048; x f32 or bf16, y f32 or bf16, not bf16 -> f32).  weight / bias f32 [d]
 * (bias may be NULL).  Writes rstd f32 [R] and, for LayerNorm, mean f32 [R] for the backward. */
int moc_row_norm_fwd(int norm, int x_dtype, const void* x, int64_t R, int64_t d, const float* weight,
                     const float* bias, float eps, int y_dtype, void* y, float* mean, float* rstd,
                     hipStream_t stream);
/* dx [R][d] and dweight_dbias f32 [2][d] = {sum_rows dy xh, sum_rows dy} (fixed order) from x,
 * the saved mean / rstd and dy.  dtypes (x, dy, dx): (f32, f32, f32), (f32, bf16, f32) or
 * (bf16, bf16, bf16). */
size_t moc_row_norm_bwd_workspace(int64_t R, int64_t d);
int moc_row_norm_bwd(int norm, int x_dtype, const void* x, int64_t R, int64_t d, const float* weight,
                     const float* mean, const float* rstd, int dy_dtype, const void* dy, int dx_dtype, void* dx,
                     float* dweight_dbias, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------ bank optimizer */

/* torch.optim.AdamW as the reference steps the bank (training/trainer.py:309-392, param group
 * "memory_bank"; torch >= 2.0 foreach algorithm, amsgrad off) for an f32 bank of num_chapters
 * chapter blocks of chunk_elems = T * d contiguous elements, optionally mirrored to a bf16 copy
 * (mirror_dtype MOC_BF16) that the forward kernels read.  Per element and step j:
 *   p = p (1 - lr_j wd); m = lerp(m, g, 1 - beta1); v = v beta2 + (1 - beta2) g g;
 *   p = p + (-lr_j / bc1_j) m / (sqrt(v) / sqrt(bc2_j) + eps).
 * Each chunk of a chapter block carries in tags i32 [num_chapters * moc_bank_chunk_count] the
 * step it is current to; hist f32 [hist_capacity][4] holds per step j the scalars
 * {1 - lr_j wd, -lr_j / bc1_j, sqrt(bc2_j), 0}.
 * grad != NULL: optimizer step `step` (scalars decay / neg_step_size / bc2_sqrt, recorded into
 *   hist[step]) with gradient grad * grad_scale[0] (grad_scale may be NULL) on the listed chapters
 *   (list i32, n_list[0] of them, at most max_list; NULL list = every chapter, dense), each chunk
 *   first brought to step-1 with zero-gradient steps.
 * grad == NULL: bring the listed chapters to `step` (zero-gradient steps from hist) — run before
 *   chapters are read.  Rows outside the list are left as they are (they are behind, exactly by
 *   their zero-gradient steps). */
int moc_bank_chunk_count(int64_t chunk_elems);
int moc_bank_adamw(float* param, void* mirror, int mirror_dtype, float* exp_avg, float* exp_avg_sq, const float* grad,
                   const float* grad_scale, const int32_t* list, const int32_t* n_list, int64_t max_list,
                   int64_t num_chapters, int64_t chunk_elems, int32_t* tags, float* hist, int64_t hist_capacity,
                   int step, float decay, float neg_step_size, float bc2_sqrt, float beta1, float beta2, float eps,
                   hipStream_t stream);
/* list = the chapters whose chap_epoch equals epoch, ascending; n_list[0] = their number. */
int moc_bank_touched(const int32_t* chap_epoch, int64_t num_chapters, int epoch, int32_t* list, int32_t* n_list,
                     hipStream_t stream);
/* out[0] = sum of g^2 over the listed chapters' blocks (NULL list: the first max_list chapters),
 * fixed order.  Feeds the global norm of clip_grad_norm_ (trainer.py:876-882). */
size_t moc_bank_sqnorm_workspace(int64_t max_list, int64_t chunk_elems);
int moc_bank_sqnorm(const float* grad, const int32_t* list, const int32_t* n_list, int64_t max_list,
                    int64_t chunk_elems, void* workspace, size_t workspace_bytes, float* out, hipStream_t stream);

/* -------------------------------------------- token-routed sparse attention */

/* Token-level routing (every query token picks its own chapters): the per-chapter
 * MoE combine of kernels-final/kernel_v4.py (FSA_topk_sparse_attention_weighted_bthd,
 * :1313-1340, and the per-chapter loop of memory_attention.py:596-688), the joint softmax
 * of kernel_v2.py (FSA_topk_sparse_attention_bthd, :3181-3315, optional block weights,
 * :765-773) and the joint log-bias of kernel_v5.py (:819-846).  Chapter-centric over a
 * chapter plan of the edges e = token * S + slot (token = b * Tq + t).
 * q [tokens][HQ][64]; K/V addressed by element strides (chapter cs, kv head hs, row rs).
 * Heads hk0 .. hk0+nhk-1 are processed; each edge serves rpe rows (query heads
 * hq_off .. hq_off+rpe-1).  Partials: o_part [E * rpe][64] in the call's dtype (bf16 or f32:
 * the per-edge rows are normalised, so bf16 keeps their round trip through HBM at half the
 * bytes), lse_part f32 [E * rpe].  bf16 runs one wave per (chapter, kv head) and needs 16-byte
 * aligned q / k / v / o_part and cs / hs / rs multiples of 8. */
int moc_sparse_fwd(int dtype, const void* q, int64_t ntok, int HQ, const void* k, const void* v, int64_t cs,
                   int64_t hs, int64_t rs, int HK, int Dh, const int32_t* uniq, const int32_t* n_uniq,
                   const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u, int S, int hk0, int nhk,
                   int hq_off, int rpe, float scale, void* o_part, float* lse_part, hipStream_t stream);
/* Combine of the slot partials: mode 0 MoE sum_s w_s o_s; 1 joint; 2 joint with block weights
 * max(w, 0); 3 joint with log(max(w, 1e-20)) bias.  w f32 [E] (per edge), edge_u from the plan
 * (negative = skipped slot), o_part in the call's dtype.  out [tokens][HQ][64]; lse_joint f32
 * [tokens * rpe] (modes 1-3).  o_part and out 16-byte aligned.  Up to 16384 rows of at most 68
 * slots (decode) take a kernel that issues every load of a row in one round. */
int moc_sparse_combine(int dtype, const void* o_part, const float* lse_part, const int32_t* edge_u, const float* w,
                       int mode, int S, int rpe, int64_t ntok, int HQ, int hq_off, void* out, float* lse_joint,
                       hipStream_t stream);
/* Backward prep: modes 1-3 -> dst f32 [tokens * rpe] = dout . out (the joint softmax delta that
 * moc_sparse_bwd reads).  mode 0 -> dst f32 [E * rpe] = dout . o_part; moc_sparse_bwd computes
 * these per-chapter deltas itself, so mode 0 callers do not need this call. */
int moc_sparse_bwd_prep(int dtype, const void* dout, const void* out, const void* o_part, const int32_t* edge_u,
                        int mode, int S, int rpe, int64_t ntok, int HQ, int hq_off, float* dst, hipStream_t stream);
/* Chapter-centric backward: dK/dV of every (chapter, kv head) stored with element strides
 * (ocs, ohs, ors) into dk / dv (rows of untouched chapters are left as they are); per-edge
 * dq parts [E * rpe][64] in the call's dtype; dlog f32 [E * rpe] (modes 2-3, d loss / d log weight).
 * delta_row: modes 1-3 read the joint delta [tokens * rpe] of moc_sparse_bwd_prep; mode 0
 * WRITES the per-chapter delta dout . o_s [E * rpe] (computed from P and dO V^T), the input
 * of moc_sparse_dw.  bf16 runs two waves per (chapter, kv head) and needs 16-byte aligned
 * q / dout / k / v / dq_part / dk / dv and cs / hs / rs / ocs / ohs / ors multiples of 8.  row_tab (bf16 only, may be NULL): moc_plan_row_table of width
 * 32 over this plan; a unit then reads its first block's edges from it together with its plan
 * entries instead of after them. */
int moc_sparse_bwd(int dtype, const void* q, const void* dout, int64_t ntok, int HQ, const void* k, const void* v,
                   int64_t cs, int64_t hs, int64_t rs, int HK, int Dh, const int32_t* uniq, const int32_t* n_uniq,
                   const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u, int S, int hk0, int nhk,
                   int hq_off, int rpe, int mode, const float* lse_row, float* delta_row, const float* w,
                   float scale, void* dk, void* dv, int64_t ocs, int64_t ohs, int64_t ors, void* dq_part,
                   float* dlog, const int32_t* row_tab, hipStream_t stream);
/* dq [tokens][HQ][64] rows hq_off .. hq_off+rpe-1 = sum over valid slots of dq_part (both 16-byte
 * aligned). */
int moc_sparse_dq_combine(int dtype, const void* dq_part, const int32_t* edge_u, int S, int rpe, int64_t ntok,
                          int HQ, int hq_off, void* dq, hipStream_t stream);
/* dw f32 [E]: mode 0 sum of dst rows; modes 2/3 sum of dlog rows / w (0 where the clamp is active). */
int moc_sparse_dw(const float* src, const float* w, const int32_t* edge_u, int mode, int rpe, int64_t E, float* dw,
                  hipStream_t stream);
/* Zeros the (chapter, kv head) blocks of dK / dV (element (t, dh) at c*cs + hk*hs + t*rs + dh,
 * heads hk0 .. hk0+nhk-1, C chapters) whose chapter is not among the plan's uniq[0 .. n_uniq):
 * moc_sparse_bwd writes every block it touches whole, so this replaces zero-initialising the
 * gradient (autograd's zeros for the unselected chapters of the reference's gather,
 * memory_bank.py:287-291).  mark i32 [C] is scratch. */
int moc_sparse_zero_untouched(int dtype, void* dk, void* dv, int64_t cs, int64_t hs, int64_t rs, int64_t C, int hk0,
                              int nhk, const int32_t* uniq, const int32_t* n_uniq, int64_t max_u, int32_t* mark,
                              hipStream_t stream);

/* ------------------------------------------------------------------ decode */

/* One decode step (L = 1) of the sequence-routed layer over precomputed per-layer K/V
 * chapter tiles of every chapter (kv_project over all chapters), i.e. the decode use of
 * memory_transformer/model.py:612-692 with the chapters and omega fixed for the generation.
 * Chapter-centric over the plan of the (sequence, slot) edges, so each selected tile is read
 * once per step.  q [B][H][64]; k_tiles, v_tiles [C][HK][64 keys][64 dims] (kv_project's
 * "k" / "v" layouts); omega f32 [B * NS], >= 0; partials o_part [B * NS * H][64] (call dtype) and
 * lse_part f32 [B * NS * H] are merged by moc_sparse_combine in joint mode (rpe = H).
 * bf16 needs 16-byte aligned q / tiles / o_part. */
int moc_decode_partial(int dtype, const void* q, int64_t B, int H, const void* k_tiles, const void* v_tiles, int HK,
                       int Dh, int T, const int32_t* uniq, const int32_t* n_uniq, const int32_t* csr_off,
                       const int32_t* csr_edge, int64_t max_u, const float* omega, int NS, float scale, void* o_part,
                       float* lse_part, const int32_t* row_tab, hipStream_t stream);
/* The decode step's row table, built once per routing: row_tab i32 [max_u][16] = the first 16
 * edges (csr order) of each distinct chapter of the plan, -1 padded (no reference counterpart: a
 * precomputed index of the same plan).  moc_decode_partial reads it (when non-NULL) instead of
 * csr_edge for a unit's first 16 rows. */
/* The same index of any width: row_tab i32 [max_u][width] = the first `width` edges (csr order) of
 * each distinct chapter, -1 padded; width 16 (moc_decode_partial) or 32 (moc_sparse_bwd). */
int moc_plan_row_table(const int32_t* n_uniq, const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u,
                       int width, int32_t* row_tab, hipStream_t stream);
int moc_decode_row_table(const int32_t* n_uniq, const int32_t* csr_off, const int32_t* csr_edge, int64_t max_u,
                         int32_t* row_tab, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MOC_H */
