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
// Largest k_slots the selection kernel sorts (k_max = 112 gives 448).
constexpr int kMaxSlots = 512;

hipError_t launch_block_summary(const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                int B, int Hk, int N, int D, int mode, uint16_t* planes,
                                hipStream_t stream);

// Outputs of the selection kernel's dump mode (on != 0): per-tile order
// statistics of the unforced tile scores, ranked k_slots = rho_k + 1 deep.
struct SelectDump {
  float* g = nullptr;        // [B, H, Qt] s(k_b - 1) - s(k_b)
  float* r = nullptr;        // [B, H, Qt] max(s(0) - s(k_b), 1e-9)
  float* sigma = nullptr;    // [B, H, Qt] clamp(g / r, 0, 2)
  float* g_rho = nullptr;    // [B, H, Qt] s(rho_k - 1) - s(rho_k)
  uint8_t* valid = nullptr;  // [Qt] visible blocks > rho_k
  int k_b = 0, rho_k = 0, on = 0;
};

hipError_t launch_select(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                         const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                         int mode, float scaling, int k_base, int k_slots, int want_sigma,
                         int32_t* kv_idx, float* sigma, float* tile_score,
                         hipStream_t stream, const SelectDump* dump = nullptr);

// Per-(b, h) score-noise estimate tau_hat of the score dump.
hipError_t launch_score_tau(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                            const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                            int mode, float scaling, float* tau_hat, hipStream_t stream);

hipError_t launch_router(const float* sigma, int B, int H, int Qt, int grain, int rmode,
                         float tau, int64_t k_quant, int32_t* kv_idx, int k_base, int k_slots,
                         int NB, float* sigma_eff, uint8_t* uncertain, float* threshold,
                         hipStream_t stream);

hipError_t launch_attn_prepare(const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                               const uint16_t* v, int64_t sv_b, int64_t sv_h, int64_t sv_n,
                               int B, int Hk, int N, int D, int block_m, uint16_t* ws,
                               hipStream_t stream);

hipError_t launch_attn_fwd(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                           const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                           const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                           int64_t si_h, int64_t si_t, int B, int H, int Hk, int M, int N,
                           int D, int Qt, int k_slots, int block_m, float scale, uint16_t* out,
                           int64_t so_b, int64_t so_h, int64_t so_m, hipStream_t stream);

}  // namespace ugbsa
