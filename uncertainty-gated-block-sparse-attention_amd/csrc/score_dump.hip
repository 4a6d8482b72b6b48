// Score-noise estimate of the score dump (tau_hat per (b, h)).
//
// Restates src/dump_block_scores.py:181-194 of the reference: for
// n_pairs = min(1024, M - 1) adjacent query-row pairs (i, i + 1) with
// i = min(p * max(1, (M - 1) / n_pairs), M - 2), the per-row block scores
// S[i, blk] (the selection's row score of :638-648, over every one of the NB
// blocks, no causal mask) give
//     tau_hat = sqrt(max(0, 0.5 * mean_{pairs, blk} (S[i + 1, blk] - S[i, blk])^2)),
// and 0 when M < 2.
//
// One workgroup per (b, h), kTauWaves wavefronts.  A wave takes 8 * MT pairs
// at a time as an MFMA A operand of 16 * MT rows ordered (lo, hi) per pair,
// so that a 16 x 16 accumulator tile holds a pair's two rows in lane
// elements (0, 1) and (2, 3): the differences need no lane exchange.  The
// KV head's summary planes stream from L2 as B operands, 16 blocks per step
// (mean planes: fp16 Q scaled per wave pass and the blocks' scales undone on
// the sums, as in the selection kernel).
// Squares are summed per lane in fp64, then over lanes and waves in a fixed
// order, so the result is deterministic.
#include "common.h"
#include "launch.h"

namespace ugbsa {

constexpr int kTauWaves = 8;
constexpr int kTauMaxPairs = 1024;   // n_pairs cap of the reference

template <typename E, int D, bool QUEST, int MT>
__global__ __launch_bounds__(64 * kTauWaves) void score_tau_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ planes, const float* __restrict__ bscale, int Hk, int M, int NB,
    int grp, int n_pairs, int stride, float scaling, float* __restrict__ tau_hat) {
  constexpr int KS = D / 32;
  constexpr int P = 2;
  constexpr int QSETS = QUEST ? 2 : 1;
  using EM = std::conditional_t<QUEST, E, ElemF16>;
  constexpr int PAIRS = 8 * MT;                     // pairs per pass
  __shared__ double part[kTauWaves];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int bh = blockIdx.x;
  const int H = Hk * grp;
  const int b = bh / H, h = bh % H;
  const uint16_t* qb = q + b * sq_b + h * sq_h;
  const uint16_t* pl = planes + (static_cast<int64_t>(b) * Hk + h / grp) * NB * P * D;
  const float* bs = QUEST ? nullptr : bscale + (static_cast<int64_t>(b) * Hk + h / grp) * NB;

  double sum = 0.0;
  const int n_pass = (n_pairs + PAIRS - 1) / PAIRS;
  for (int pass = wave; pass < n_pass; pass += kTauWaves) {
    bf16x8 qf[QSETS][MT][KS];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int pair = pass * PAIRS + 8 * mt + (r16 >> 1);
      const bool live = pair < n_pairs;
      int row = min(pair * stride, M - 2) + (r16 & 1);
      row = live ? row : 0;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 x = live ? load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4) : zero_bf16x8();
        if constexpr (QUEST) {
          qf[0][mt][ks] = bf16_pos(x);
          qf[QSETS - 1][mt][ks] = bf16_neg(x);
        } else {
          qf[0][mt][ks] = x;
        }
      }
    }
    float tdesc = 1.f;
    if constexpr (!QUEST) tdesc = q_tile_to_f16<E, MT * KS>(&qf[0][0][0], lane);
    for (int n0 = 0; n0 < NB; n0 += 16) {
      const int blk = n0 + r16;
      f32x4 acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < P; ++p) {
        bf16x8 bfr[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          bfr[ks] = blk < NB ? load_bf16x8(pl + static_cast<int64_t>(blk) * P * D + p * D +
                                           32 * ks + 8 * g4)
                             : zero_bf16x8();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt] = EM::mfma(qf[QUEST ? p : 0][mt][ks], bfr[ks], acc[mt]);
      }
      // the exact factor from the sums to the scores of this lane's block
      const float cs = QUEST ? 1.f : (blk < NB ? bs[blk] : 0.f) * tdesc;
      // rows (4 g4 + 0, 4 g4 + 1) and (4 g4 + 2, 4 g4 + 3) are (lo, hi) of
      // two pairs; dead pairs and blocks past NB score 0 on both rows
      float s2 = 0.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float d0 = (acc[mt][1] * cs) * scaling - (acc[mt][0] * cs) * scaling;
        const float d1 = (acc[mt][3] * cs) * scaling - (acc[mt][2] * cs) * scaling;
        s2 += d0 * d0 + d1 * d1;
      }
      sum += static_cast<double>(s2);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
  if (lane == 0) part[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
    for (int w = 0; w < kTauWaves; ++w) tot += part[w];
    float tau = 0.f;
    if (n_pairs > 0) {
      const float mean = static_cast<float>(tot / (static_cast<double>(n_pairs) * NB));
      const float tsq = 0.5f * mean;
      tau = sqrtf(tsq > 0.f ? tsq : 0.f);
    }
    tau_hat[bh] = tau;
  }
}

template <typename E, int D, bool QUEST>
static hipError_t launch_tau_t(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                               const uint16_t* planes, int B, int H, int Hk, int M, int N,
                               float scaling, float* tau_hat, hipStream_t stream) {
  // A operands of 4 m-tiles while they fit in 128 VGPRs, else 2
  constexpr int MT = (QUEST ? 2 : 1) * 4 * (D / 32) * 4 <= 128 ? 4 : 2;
  const int NB = (N + kBlock - 1) / kBlock;
  const int n_pairs = M >= 2 ? (M - 1 < kTauMaxPairs ? M - 1 : kTauMaxPairs) : 0;
  const int stride = n_pairs > 0 ? ((M - 1) / n_pairs > 1 ? (M - 1) / n_pairs : 1) : 1;
  score_tau_kernel<E, D, QUEST, MT><<<dim3(static_cast<unsigned>(B * H)), 64 * kTauWaves, 0, stream>>>(
      q, sq_b, sq_h, sq_m, planes, QUEST ? nullptr : mean_descale(planes, B, Hk, NB, D), Hk, M,
      NB, H / Hk, n_pairs, stride, scaling, tau_hat);
  return hipGetLastError();
}

template <typename E>
static hipError_t launch_score_tau_e(const uint16_t* q, int64_t sq_b, int64_t sq_h,
                                     int64_t sq_m, const uint16_t* planes, int B, int H, int Hk,
                                     int M, int N, int D, int mode, float scaling,
                                     float* tau_hat, hipStream_t stream) {
  const bool quest = mode == kModeQuest;
#define UGBSA_TAU(D_)                                                                          \
  return quest ? launch_tau_t<E, D_, true>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, scaling,   \
                                        tau_hat, stream)                                        \
               : launch_tau_t<E, D_, false>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, scaling,   \
                                        tau_hat, stream)
  if (D == 64) UGBSA_TAU(64);
  if (D == 128) UGBSA_TAU(128);
  if (D == 256) UGBSA_TAU(256);
#undef UGBSA_TAU
  return hipErrorInvalidValue;
}

hipError_t launch_score_tau(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                            const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                            int elem, int mode, float scaling, float* tau_hat,
                            hipStream_t stream) {
  if (elem == ElemF16::code)
    return launch_score_tau_e<ElemF16>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, D, mode,
                                       scaling, tau_hat, stream);
  return launch_score_tau_e<ElemBf16>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, D, mode,
                                      scaling, tau_hat, stream);
}

}  // namespace ugbsa
