// Internal launcher declarations shared by the kernel files and the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ugbsa {

// Block-score backbone (Selector.router_score / mode).
constexpr int kModeMean = 0;
constexpr int kModeQuest = 1;

// Router knobs (Selector.router_grain / router_mode).
constexpr int kGrainCell = 0;
constexpr int kGrainRow = 1;
constexpr int kRouterAbs = 0;
constexpr int kRouterQuantile = 1;

// Largest key-block count the selection kernel keeps in LDS per head: a
// wave's fp32 score row takes 4 * NB bytes, 64 KiB at 16384 blocks (1M
// tokens), where one wave per workgroup still fits beside the chunk buffers.
constexpr int kMaxBlocksSelect = 16384;
// Largest key-block count of the per-row (v1) selector: one fp32 row of
// scores per wavefront in LDS.
constexpr int kStreamBlocksRows = 4096;
// Largest k_slots the selection kernel sorts (k_max = 112 gives 448).
constexpr int kMaxSlots = 512;

// elem: the 16-bit element format of the call's tensors (ElemBf16::code 0 or
// ElemF16::code 1, the C ABI's UGBSA_DTYPE_* values).
hipError_t launch_block_summary(const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                int B, int Hk, int N, int D, int elem, int mode,
                                uint16_t* planes, hipStream_t stream);

// Extra modes of the selection kernel.
//  dump != 0: per-tile order statistics of the unforced tile scores, ranked
//             k_slots = rho_k + 1 deep, written instead of kv_idx;
//  row_scores != nullptr: the per-row scores of tiles [rows_t0, rows_t1)
//             (rows past M skipped) into row_scores [B, H, 64 * (rows_t1 -
//             rows_t0), NB] fp32, -inf past each tile's visible blocks, and
//             nothing else (the v1 per-row selector's input).
struct SelectAux {
  float* g = nullptr;        // [B, H, Qt] s(k_b - 1) - s(k_b)
  float* r = nullptr;        // [B, H, Qt] max(s(0) - s(k_b), 1e-9)
  float* sigma = nullptr;    // [B, H, Qt] clamp(g / r, 0, 2)
  float* g_rho = nullptr;    // [B, H, Qt] s(rho_k - 1) - s(rho_k)
  uint8_t* valid = nullptr;  // [Qt] visible blocks > rho_k
  int k_b = 0, rho_k = 0, dump = 0;
  float* row_scores = nullptr;
  int rows_t0 = 0, rows_t1 = 0;
};

hipError_t launch_select(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                         const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                         int elem, int mode, float scaling, int k_base, int k_slots,
                         int want_sigma, int32_t* kv_idx, float* sigma, float* tile_score,
                         hipStream_t stream, const SelectAux* aux = nullptr);

// The v1 per-row selector over a buffer of per-row scores (SelectAux
// row_scores): one wavefront per row ranks its visible blocks K deep and
// writes the row's keep bytes (the k_bud best, or the belief budget's best,
// plus the sink and the row's own block) and, with k_eff > 0, its margin.
struct RowsArgs {
  const float* scores = nullptr;   // [B, H, nrows, NB]: rows r0 .. r0 + nrows - 1
  int r0 = 0, nrows = 0;
  int B = 0, H = 0, M = 0, NB = 0;
  int K = 0;                       // ranked depth (<= 512, <= NB)
  int k_bud = 0;                   // blocks kept per row (top-k family)
  int belief = 0;                  // 1: budget from the top_p softmax mass
  float top_p = 0.f;
  int k_min = 0, k_max = 0;
  int k_eff = 0;                   // router margin at rank k_eff (0: none)
  const float* penalty = nullptr;  // [H, NB] subtracted from row M - 1 (rollout)
  uint8_t* keep = nullptr;         // [B, H, M, NB]
  float* margin = nullptr;         // [B, H, M]
};

hipError_t launch_select_rows(const RowsArgs& a, hipStream_t stream);

// Per-(b, h) score-noise estimate tau_hat of the score dump.
hipError_t launch_score_tau(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                            const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                            int elem, int mode, float scaling, float* tau_hat,
                            hipStream_t stream);

hipError_t launch_router(const float* sigma, int B, int H, int Qt, int grain, int rmode,
                         float tau, int64_t k_quant, int32_t* kv_idx, int k_base, int k_slots,
                         int NB, float* sigma_eff, uint8_t* uncertain, float* threshold,
                         hipStream_t stream);

// v1 router: threshold over the rows' margins, trigger flags, and the keep
// rows of uncertain cells set to their visible blocks.  threshold must be a
// device float (the fill kernel reads it).
hipError_t launch_router_rows(const float* margin, int B, int H, int M, int NB, int grain,
                              int rmode, float tau, int64_t k_quant, int elig_row0,
                              uint8_t* keep, float* margin_eff, uint8_t* uncertain,
                              float* threshold, hipStream_t stream);

hipError_t launch_attn_prepare(const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                               const uint16_t* v, int64_t sv_b, int64_t sv_h, int64_t sv_n,
                               int B, int Hk, int N, int D, int block_m, uint16_t* ws,
                               hipStream_t stream);

hipError_t launch_attn_fwd(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                           const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                           const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                           int64_t si_h, int64_t si_t, int B, int H, int Hk, int M, int N,
                           int D, int elem, int Qt, int k_slots, int block_m, float scale,
                           uint16_t* out, int64_t so_b, int64_t so_h, int64_t so_m,
                           hipStream_t stream, const uint64_t* rowmask = nullptr,
                           int32_t* order_ws = nullptr);

// The (b, t) tiles of a kv_idx [B, H, Qt, k_slots] ordered by their visited
// slots over all query heads, heaviest first (64-row tiles): ws holds 2 * B *
// Qt int32 — the per-tile work, then the order (b * Qt + t per entry).
hipError_t launch_attn_tile_order(const int32_t* kv_idx, int64_t si_b, int64_t si_h,
                                  int64_t si_t, int B, int H, int Qt, int k_slots, int NB,
                                  int32_t* ws, hipStream_t stream);

// The pipelined attention kernel at head_dim 256 (attn_fwd256.hip: one
// wavefront per 64-row tile, O^T in AGPRs, Q in LDS, one K / V^T set).
hipError_t launch_attn_pipe256(int elem, const uint16_t* q, int64_t sq_b, int64_t sq_h,
                               int64_t sq_m,
                               const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                               const uint16_t* vt, const int32_t* kv_idx,
                               const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                               int64_t si_t, int B, int H, int Hk, int M, int N, int Qt,
                               int k_slots, float scale, uint16_t* out, int64_t so_b,
                               int64_t so_h, int64_t so_m, hipStream_t stream,
                               const int32_t* tile_order);

// _compute_kv_idx on the GPU: per (b, h, block_m-row tile) the blocks any row
// of keep [B, H, M, NB] (uint8, contiguous) keeps, ascending, NB-padded to
// NB slots, their count, and (if rowmask) each listed block's row mask.
hipError_t launch_keep_kv_idx(const uint8_t* keep, int B, int H, int M, int NB, int block_m,
                              int32_t* kv_idx, uint64_t* rowmask, int32_t* counts,
                              hipStream_t stream);

}  // namespace ugbsa
