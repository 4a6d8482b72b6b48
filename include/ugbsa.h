/* libugbsa — C ABI of the MI355X (gfx950) sparse-prefill hot path.
 *
 * The reference implements this path as Python/torch + Triton inside
 * src/sparse_attention.py (_block_select_kv_idx_v2, :588-748) and
 * src/triton_block_attn.py (block_sparse_attn_v2, :267-298, kernel :184-264).
 * Each entry point below replaces one of those pieces; the Python host layer
 * (sparse_attention.py / block_attn.py in the package) calls them through
 * ctypes with torch-owned device pointers.
 *
 * Conventions
 *  - Pointers are device pointers (e.g. torch.Tensor.data_ptr()); the library
 *    never allocates or frees device memory and keeps no pointer after return.
 *  - Strides are in elements (int64).  The 16-bit tensors of a call (q, k, v,
 *    the Quest summary planes, out) share one element format, `dtype`
 *    (the mean summary is fp16 and fp32 for both, see ugbsa_block_summary):
 *    UGBSA_DTYPE_BF16 or UGBSA_DTYPE_F16 — the reference runs in the model's
 *    dtype (src/triton_block_attn.py:267-298, src/sparse_attention.py:588-748).
 *    They need head_dim stride 1, 16-byte aligned base pointers and other
 *    strides that are multiples of 8.
 *  - Every launch is asynchronous on `stream` (a hipStream_t; NULL = default
 *    stream).  No entry point synchronises the host.
 *  - Return value: 0 on success, > 0 a hipError_t from the launch, < 0 an
 *    argument error (UGBSA_E*).  ugbsa_last_error() gives a message for the
 *    calling thread's last failure.
 *  - Key blocks are 64 tokens (the reference's BLOCK, src/sparse_attention.py:51).
 */
#ifndef UGBSA_H
#define UGBSA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UGBSA_ABI_VERSION 4

#define UGBSA_OK 0
#define UGBSA_EARG (-1)     /* bad size / value / null pointer */
#define UGBSA_ELAYOUT (-2)  /* stride or alignment the kernels cannot read */
#define UGBSA_EDTYPE (-3)   /* unsupported element type */

#define UGBSA_DTYPE_BF16 0
#define UGBSA_DTYPE_F16 1

#define UGBSA_MODE_MEAN 0   /* K-mean backbone (Selector.router_score "mean", mode "topk") */
#define UGBSA_MODE_QUEST 1  /* Quest K-max/K-min backbone (mode "quest", router_score "quest") */

#define UGBSA_GRAIN_CELL 0  /* Selector.router_grain */
#define UGBSA_GRAIN_ROW 1
#define UGBSA_ROUTER_ABS 0  /* Selector.router_mode */
#define UGBSA_ROUTER_QUANTILE 1

#define UGBSA_V1_TOPK 0     /* per-row budget k_bud (modes topk, quest, router, rollout) */
#define UGBSA_V1_BELIEF 1   /* per-row budget from the top_p softmax mass (mode belief) */

int ugbsa_abi_version(void);
const char* ugbsa_last_error(void);

/* Number of 16-bit elements of the block-summary buffer: Quest
 * [B, Hk, NB, 2, D]; mean [B, Hk, NB, 2, D] fp16 followed by [B, Hk, NB] fp32
 * (B * Hk * NB * (2 * D + 2) in all). */
int64_t ugbsa_summary_elems(int B, int Hk, int N, int D, int mode);

/* Kernel 1 — per-64-token-block K summaries of k [B, Hk, N, D] (dtype).
 * Replaces the summary step of _block_select_kv_idx_v2:
 * src/sparse_attention.py:618-622 (zero pad), :636-637 (amin/amax, Quest),
 * :646 (mean).  Output: Quest, two planes in dtype (K-max, K-min, exact);
 * mean, for either dtype, two fp16 planes hi, lo with hi + lo = the block's
 * fp32 mean times 2^e to 22-23 bits (e per block, max_d |mean_d| 2^e in
 * [2^14, 2^15)), then 2^-e per block as fp32.  The mean of block blk of
 * (b, g) is (hi + lo) * scale[(b * Hk + g) * NB + blk]. */
int ugbsa_block_summary(const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                        int B, int Hk, int N, int D, int dtype, int mode, void* planes,
                        void* stream);

/* Kernel 2 — fused per-Q-tile block scoring, tile max-pool, visibility,
 * sink/self forcing, top-k_slots and (if sigma != NULL) the sigma margin.
 * Replaces src/sparse_attention.py:623-707 of _block_select_kv_idx_v2
 * (per-row scores :638-648, tile max :655-656, causal tile mask :660-666,
 * FMAX forcing :675-681, topk :697, margin :703-707).
 * q [B, H, M, D] in dtype, planes from ugbsa_block_summary of the same
 * dtype and mode (query head h uses KV head h / (H / Hk));
 * kv_idx out [B, H, Qt, k_slots] int32 contiguous, slots ordered by
 * (score desc, block asc); sigma out [B, H, Qt] fp32; tile_score (optional
 * diagnostic) out [B, H, Qt, NB] fp32 = the exact scores ranked.
 * Qt = ceil(M / 64), NB = ceil(N / 64); block_m must be 64. */
int ugbsa_select(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                 const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                 int mode, float scaling, int k_base, int k_slots, int block_m, int32_t* kv_idx,
                 float* sigma, float* tile_score, void* stream);

/* Score dump — the per-tile order statistics and per-head score-noise
 * estimate that src/dump_block_scores.py (_record, :104-207) records beside
 * each selection call, computed from kernel 1's planes by kernel 2 in dump
 * mode plus one reduction kernel.  With s(0) >= s(1) >= ... the tile's
 * scores before sink/self forcing (invisible blocks -inf, :137-147, sorted
 * :161; the gaps :162-171):
 *   g [B, H, Qt]      s(k_b - 1) - s(k_b)
 *   r [B, H, Qt]      max(s(0) - s(k_b), 1e-9)
 *   sigma [B, H, Qt]  min(max(g / r, 0), 2), NaN kept
 *   g_rho [B, H, Qt]  s(rho_k - 1) - s(rho_k)
 *   valid [Qt] uint8  visible blocks of tile t > rho_k
 *   tau_hat [B, H]    sqrt(max(0, mean over n_pairs = min(1024, M - 1) row
 *                     pairs (i, i + 1), i = min(p * max(1, (M - 1) / n_pairs),
 *                     M - 2), and all NB blocks of (S[i + 1] - S[i])^2 / 2)),
 *                     S the per-row block score; 0 when M < 2 (:181-194)
 *   tile_score        optional [B, H, Qt, NB] fp32, the unforced scores.
 * The caller passes k_b = min(2 * budget_blocks, NB), rho_k = min(2 * k_b,
 * NB) (:150-151); needs 1 <= k_b < rho_k < NB and rho_k < 512. */
int ugbsa_score_dump(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                     const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                     int mode, float scaling, int k_b, int rho_k, float* g, float* r,
                     float* sigma, float* g_rho, uint8_t* valid, float* tau_hat,
                     float* tile_score, void* stream);

/* Router — row/cell grain, quantile/abs trigger and sentinel emission.
 * Replaces src/sparse_attention.py:708-725.  k_quant = max(1, int(q * B*H*Qt))
 * computed by the caller as the reference does (:714).  Writes sigma_eff
 * [B, H, Qt] fp32 (after the head mean for row grain), uncertain [B, H, Qt]
 * uint8, the threshold (1 float, optional) and sets kv_idx[..., k_base:] = NB
 * for tiles that are not uncertain. */
int ugbsa_router(const float* sigma, int B, int H, int Qt, int grain, int rmode, float tau,
                 int64_t k_quant, int32_t* kv_idx, int k_base, int k_slots, int NB,
                 float* sigma_eff, uint8_t* uncertain, float* threshold, void* stream);

/* ---- v1 per-row path (kernel_v2=False) ---------------------------------- */

/* fp32 elements of a ugbsa_select_mask workspace that scores every row in one
 * pass ([B, H, ceil(M / 64) * 64, NB]); any multiple of B * H * 64 * NB also
 * works, processed in that many rows at a time. */
int64_t ugbsa_select_mask_workspace_elems(int B, int H, int M, int N);

/* Per-row block selection: keep [B, H, M, NB] uint8 (0/1, contiguous) of
 * _block_select_mask, src/sparse_attention.py:208-295 (the router's trigger
 * is ugbsa_router_rows).  Per query row the block scores of kernel 2's
 * backbone (-inf past the row's visible blocks, :218-244), ranked by (score
 * desc, block asc); kept: the k_bud best (policy UGBSA_V1_TOPK, :273-283) or
 * the clamp(#{cumsum of sorted softmax < top_p} + 1, k_min, k_max) best
 * (UGBSA_V1_BELIEF, :262-270, 284-285); ranks past the visible blocks keep
 * the lowest invisible blocks; then the sink and the row's own block
 * (:287-289).  penalty [H, NB] (or NULL) is subtracted from the scores of
 * row M - 1 first (rollout, :247-259).  k_eff > 0 also writes margin
 * [B, H, M] = (s[k_eff - 1] - s[k_eff]) / max(s[0] - s[k_eff], 1e-6)
 * (:299-316).  Needs M == N, NB <= 4096; the workspace holds the row scores
 * of the last pass on return. */
int ugbsa_select_mask(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                      const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                      int mode, float scaling, int policy, int k_bud, int k_eff, int k_min,
                      int k_max, float top_p, const float* penalty, float* workspace,
                      int64_t workspace_elems, uint8_t* keep, float* margin, void* stream);

/* ugbsa_select_mask without a caller workspace.  No counterpart in the
 * reference: it serves callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Arguments and results as ugbsa_select_mask; the per-row scores of each pass
 * go to a file-scope device array of 2^24 fp32 (64 MiB) per GPU, held until
 * the process ends, instead of `workspace`.  Needs B * H * 64 * NB <= 2^24 (one
 * 64-row tile per pass; larger shapes return UGBSA_EARG before any launch)
 * and calls no allocator.  Every call on a GPU shares that GPU's array, so
 * calls that overlap on one GPU (other streams, other threads) race; the
 * array keeps the last call's scores, and nothing in it needs clearing.
 * Under stream capture: make one call on the device first (it looks the
 * array's address up); a captured call then replays like a direct one. */
int ugbsa_select_mask_static(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                             int64_t sq_d, const void* planes, int B, int H, int Hk, int M, int N,
                             int D, int dtype, int mode, float scaling, int policy, int k_bud,
                             int k_eff, int k_min, int k_max, float top_p, const float* penalty,
                             uint8_t* keep, float* margin, void* stream);

/* v1 router (src/sparse_attention.py:317-354): margin_eff = margin, or its
 * head mean for row grain; rows with more than k_eff visible blocks are
 * eligible; quantile: thr = k_quant-th smallest of m_safe (margin_eff, +inf
 * where ineligible or NaN) over B * M (row) or B * H * M (cell) values,
 * uncertain = m_safe <= thr (k_quant = max(1, int(q * n_elig)) from the
 * caller, 0 when nothing is eligible); abs: uncertain = margin_eff < tau.
 * Uncertain cells' keep rows are set to their visible blocks.  threshold: a
 * device float (NaN unless quantile with k_quant > 0). */
int ugbsa_router_rows(const float* margin, int B, int H, int M, int NB, int grain, int rmode,
                      float tau, int64_t k_quant, int k_eff, uint8_t* keep, float* margin_eff,
                      uint8_t* uncertain, float* threshold, void* stream);

/* _compute_kv_idx (src/triton_block_attn.py:125-146) of keep [B, H, M, NB]
 * uint8 contiguous: kv_idx [B, H, Qt, NB] int32 — per block_m-row tile the
 * blocks any row keeps, ascending, padded with NB — counts [B, H, Qt] (the
 * caller's max is MAX_KEPT), and rowmask [B, H, Qt, NB] uint64 (or NULL):
 * per listed block the tile rows keeping it (bit r = row t * block_m + r). */
int ugbsa_keep_kv_idx(const uint8_t* keep, int B, int H, int M, int NB, int block_m,
                      int32_t* kv_idx, uint64_t* rowmask, int32_t* counts, void* stream);

/* Kernel 3 with per-row keep masks: replaces block_sparse_attn
 * (src/triton_block_attn.py:149-182) and its kernel _fwd_kernel (:39-122).
 * Arguments as ugbsa_attn_fwd, plus rowmask with kv_idx's shape and element
 * strides (ugbsa_keep_kv_idx): a row attends to a listed block's keys only
 * if its bit is set (and causally).  Slots are visited in order; k_slots <=
 * 8192 for head_dim <= 128 with 64-row tiles. */
int ugbsa_attn_fwd_rows(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                        const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                        const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                        const int32_t* kv_idx, const uint64_t* rowmask, int64_t si_b,
                        int64_t si_h, int64_t si_t, int64_t si_s, int B, int H, int Hk, int M,
                        int N, int D, int dtype, int Qt, int k_slots, int block_m, float scale,
                        void* out, int64_t so_b, int64_t so_h, int64_t so_m, int64_t so_d,
                        void* workspace, int64_t workspace_elems, void* stream);

/* Number of 16-bit elements of the attention workspace, in two parts:
 *   1. the K and V operand copies written by ugbsa_attn_prepare_kv,
 *      2 * B * Hk * NB * 64 * D elements (NB = ceil(N / 64));
 *   2. the tile schedule ugbsa_attn_fwd / ugbsa_attn_fwd_rows write before
 *      their launches: 2 * B * NB int32 (per-tile work, then the tile order),
 *      i.e. 4 * B * NB elements rounded up to a multiple of 8 (16 bytes).
 * ugbsa_attn_prepare_kv needs only part 1; the attention entry points need
 * both and reject a smaller workspace_elems with UGBSA_EARG. */
int64_t ugbsa_attn_workspace_elems(int B, int Hk, int N, int D);

/* K and V of every 64-key block re-laid in the attention kernel's operand
 * order (for block_m 64 at head_dim 64/128: K and V^T as 1 KiB per-lane slabs
 * per 32-key half block; otherwise V^T per block), keys past N zero.  Part of
 * block_sparse_attn_v2's work (src/triton_block_attn.py:267-298), exposed so
 * a caller can prepare K/V once and time or reuse it.  workspace_elems: the
 * 16-bit elements the caller's workspace holds, at least part 1 of
 * ugbsa_attn_workspace_elems (UGBSA_EARG otherwise). */
int ugbsa_attn_prepare_kv(const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                          const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                          int B, int Hk, int N, int D, int dtype, int block_m, void* workspace,
                          int64_t workspace_elems, void* stream);

/* Kernel 3 — block-sparse causal attention over kv_idx.
 * Replaces block_sparse_attn_v2 (src/triton_block_attn.py:267-298) and its
 * kernel _fwd_kernel_v2 (:184-264).  q [B, H, M, D], k/v [B, Hk, N, D] in dtype
 * (Hk may equal H, as after repeat_kv), kv_idx [B, H, Qt, k_slots] int32 with
 * Qt = ceil(M / block_m), block_m 64 or 32, sentinel NB skipped; out
 * [B, H, M, D] in dtype (P rounded to dtype before P.V, as the reference's
 * p.to(v.dtype)) with arbitrary strides (head_dim stride 1).  v may be
 * NULL when workspace already holds ugbsa_attn_prepare_kv(k, v, block_m);
 * otherwise the preparation runs first, on the same stream.  workspace holds
 * workspace_elems 16-bit elements, at least ugbsa_attn_workspace_elems(B, Hk,
 * N, D): the K/V operand copies, then the tile schedule, which every call
 * rewrites (UGBSA_EARG before any launch if it is smaller).  scale must be
 * finite and nonzero (UGBSA_EARG otherwise). */
int ugbsa_attn_fwd(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                   const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                   const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                   const int32_t* kv_idx, int64_t si_b, int64_t si_h, int64_t si_t,
                   int64_t si_s, int B, int H, int Hk, int M, int N, int D, int dtype, int Qt,
                   int k_slots, int block_m, float scale, void* out, int64_t so_b,
                   int64_t so_h, int64_t so_m, int64_t so_d, void* workspace,
                   int64_t workspace_elems, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UGBSA_H */
