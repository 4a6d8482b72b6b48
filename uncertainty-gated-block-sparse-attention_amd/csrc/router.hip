// Router pass: sigma -> per-layer trigger decision -> sentinel fill of kv_idx.
//
// Restates src/sparse_attention.py:708-725:
//   row grain   sigma_eff[b, :, t] = (sum_h sigma[b, h, t]) / H   (fp32, heads in
//               order; ATen's CPU mean is sum then divide);
//   quantile    thr = k_quant-th smallest of sigma_eff over all (b, h, t), NaN
//               ranked above every number (torch.kthvalue); uncertain = eff <= thr;
//   abs         uncertain = eff < tau;
//   emission    kv_idx[b, h, t, k_base:] = NB where not uncertain.
// k_quant = max(1, int(q * B * H * Qt)) is computed by the host, as the
// reference does in Python.  With row grain every tile's mean appears H
// times in the flattened tensor, so its k_quant-th smallest is the
// ((k_quant - 1) / H + 1)-th smallest per-tile mean.
//
// The threshold needs every tile's sigma, so it runs as one 1024-thread
// workgroup (an 8-bit radix select, 4 passes), followed by a grid-wide fill.
// With row grain the per-tile head means stay in LDS while B * Qt <=
// kRouterLdsMeans (every BASELINE shape, 1M tokens included), so the radix
// passes and the decisions read LDS rather than L2; larger inputs and cell
// grain select over sigma_eff in global memory.
#include "common.h"
#include "launch.h"

namespace ugbsa {

// Sum over h = 0 .. H-1 of x[h * stride], added in head order (the order of
// ATen's CPU sum that the reference's mean runs), with the loads issued NL
// at a time so that their latencies overlap.
template <int NL = 8>
__device__ __forceinline__ float head_sum_in_order(const float* __restrict__ x, int H,
                                                   int64_t stride) {
  float acc = 0.f;
  for (int h0 = 0; h0 < H; h0 += NL) {
    float v[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) v[j] = h0 + j < H ? x[(h0 + j) * stride] : 0.f;
#pragma unroll
    for (int j = 0; j < NL; ++j)
      if (h0 + j < H) acc = h0 + j == 0 ? v[0] : acc + v[j];
  }
  return acc;
}

constexpr int kRouterLdsMeans = 16384;   // per-tile means held in LDS (64 KiB)

// k-th smallest (1-based) of value_at(0 .. n - 1) by one workgroup: a
// 4-pass 8-bit radix select over the order-preserving float keys (NaN above
// every number); returns the key to every thread.  Each wavefront counts
// into its own 256-bin histogram (hist holds kRouterWaves of them): the keys
// of one pass mostly share their top digits, and one shared histogram would
// serialise the LDS atomics of the whole workgroup on a few bins.
constexpr int kRouterWaves = 16;   // 1024-thread workgroups
template <class F>
__device__ uint32_t block_kth_smallest(F value_at, int64_t n, int64_t kth, uint32_t* hist,
                                       uint32_t* s_prefix, uint32_t* s_remaining) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int wave = tid >> 6;
  uint32_t* whist = hist + wave * 256;
  if (tid == 0) { *s_prefix = 0; *s_remaining = static_cast<uint32_t>(kth); }
  uint32_t pmask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256 * kRouterWaves; i += nt) hist[i] = 0;
    __syncthreads();
    const uint32_t prefix = *s_prefix;
    for (int64_t i = tid; i < n; i += nt) {
      const uint32_t key = float_key(value_at(i));
      if ((key & pmask) == prefix) atomicAdd(&whist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 256) {   // fold the per-wave histograms into the first
      uint32_t c = 0;
      for (int w = 0; w < kRouterWaves; ++w) c += hist[w * 256 + tid];
      hist[tid] = c;
    }
    __syncthreads();
    if (tid < 64) {
      // ascending scan for the bin holding the remaining-th smallest: lane L
      // owns bins 4L .. 4L + 3, a wavefront prefix sum over the lane totals
      // finds the lane, the lane walks its four bins
      const uint32_t rem = *s_remaining;
      const uint32_t h0 = hist[4 * tid], h1 = hist[4 * tid + 1];
      const uint32_t h2 = hist[4 * tid + 2], h3 = hist[4 * tid + 3];
      const uint32_t below = wave_excl_scan(h0 + h1 + h2 + h3, tid);
      const bool hit = below < rem && below + h0 + h1 + h2 + h3 >= rem;
      if (hit) {   // exactly one lane: the counts are cumulative and rem <= total
        uint32_t at = below;
        int d = 4 * tid;
        if (at + h0 < rem) { at += h0; ++d;
          if (at + h1 < rem) { at += h1; ++d;
            if (at + h2 < rem) { at += h2; ++d; } } }
        *s_prefix = prefix | (static_cast<uint32_t>(d) << shift);
        *s_remaining = rem - at;
      }
    }
    pmask |= 0xFFu << shift;
    __syncthreads();
  }
  return *s_prefix;
}

__global__ __launch_bounds__(1024) void router_threshold_kernel(
    const float* __restrict__ sigma, int B, int H, int Qt, int grain, int rmode, float tau,
    int64_t k_quant, float* __restrict__ sigma_eff, uint8_t* __restrict__ uncertain,
    float* __restrict__ threshold) {
  __shared__ uint32_t hist[256 * kRouterWaves];
  __shared__ uint32_t s_prefix, s_remaining;
  extern __shared__ float smean[];          // [B * Qt] when in_lds
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t n_all = static_cast<int64_t>(B) * H * Qt;
  const int64_t n_tiles = static_cast<int64_t>(B) * Qt;
  const bool in_lds = grain == kGrainRow && n_tiles <= kRouterLdsMeans;

  // 1. effective sigma (with in_lds, sigma_eff is written with the decisions)
  if (grain == kGrainRow) {
    for (int b = 0; b < B; ++b)
      for (int t = tid; t < Qt; t += nt) {
        const float acc =
            head_sum_in_order<32>(sigma + (static_cast<int64_t>(b) * H) * Qt + t, H, Qt);
        const float mean = acc / static_cast<float>(H);
        if (in_lds) {
          smean[b * Qt + t] = mean;
        } else {
          for (int h = 0; h < H; ++h) sigma_eff[(static_cast<int64_t>(b) * H + h) * Qt + t] = mean;
        }
      }
  } else {
    for (int64_t i = tid; i < n_all; i += nt) sigma_eff[i] = sigma[i];
  }
  __syncthreads();

  // 2. threshold
  float thr = tau;
  if (rmode == kRouterQuantile) {
    // rank among the values examined: per-tile means (row) or all cells
    const int64_t n = grain == kGrainRow ? n_tiles : n_all;
    const int64_t kth = grain == kGrainRow ? (k_quant - 1) / H + 1 : k_quant;  // 1-based
    auto value_at = [&](int64_t i) -> float {
      if (in_lds) return smean[i];
      if (grain == kGrainRow) {
        const int64_t b = i / Qt, t = i % Qt;
        return sigma_eff[(b * H) * Qt + t];
      }
      return sigma_eff[i];
    };
    thr = key_float(block_kth_smallest(value_at, n, kth, hist, &s_prefix, &s_remaining));
  }
  if (tid == 0 && threshold != nullptr) *threshold = thr;

  // 3. decision (NaN never triggers: comparisons with NaN are false)
  if (in_lds) {
    for (int bh = 0; bh < B * H; ++bh) {
      const float* mrow = smean + (bh / H) * Qt;
      const int64_t r0 = static_cast<int64_t>(bh) * Qt;
      for (int t = tid; t < Qt; t += nt) {
        const float e = mrow[t];
        sigma_eff[r0 + t] = e;
        uncertain[r0 + t] = rmode == kRouterQuantile ? (e <= thr) : (e < tau);
      }
    }
  } else {
    for (int64_t i = tid; i < n_all; i += nt) {
      const float e = sigma_eff[i];
      uncertain[i] = rmode == kRouterQuantile ? (e <= thr) : (e < tau);
    }
  }
}

// kv_idx[row, k_base:k_slots] = NB for rows that are not uncertain.
__global__ __launch_bounds__(256) void router_fill_kernel(
    int32_t* __restrict__ kv_idx, const uint8_t* __restrict__ uncertain, int64_t rows,
    int k_base, int k_slots, int NB) {
  const int extra = k_slots - k_base;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * extra) return;
  const int64_t row = i / extra;
  const int j = static_cast<int>(i % extra);
  if (!uncertain[row]) kv_idx[row * k_slots + k_base + j] = NB;
}

hipError_t launch_router(const float* sigma, int B, int H, int Qt, int grain, int rmode,
                         float tau, int64_t k_quant, int32_t* kv_idx, int k_base, int k_slots,
                         int NB, float* sigma_eff, uint8_t* uncertain, float* threshold,
                         hipStream_t stream) {
  const int64_t n_tiles = static_cast<int64_t>(B) * Qt;
  const size_t lds = grain == kGrainRow && n_tiles <= kRouterLdsMeans
                         ? static_cast<size_t>(n_tiles) * sizeof(float) : 0;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(router_threshold_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     kRouterLdsMeans * static_cast<int>(sizeof(float)));
  if (e != hipSuccess) return e;
  router_threshold_kernel<<<1, 1024, lds, stream>>>(sigma, B, H, Qt, grain, rmode, tau, k_quant,
                                                    sigma_eff, uncertain, threshold);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = static_cast<int64_t>(B) * H * Qt;
  const int64_t total = rows * (k_slots - k_base);
  if (total > 0) {
    const int64_t grid = (total + 255) / 256;
    router_fill_kernel<<<dim3(static_cast<unsigned>(grid)), 256, 0, stream>>>(
        kv_idx, uncertain, rows, k_base, k_slots, NB);
  }
  return hipGetLastError();
}

// v1 router (src/sparse_attention.py:297-354), per query row: the margins of
// the rows (select_rows_kernel), averaged over heads in order for row grain;
// rows with more than k_eff visible blocks (row >= elig_row0 = 64 k_eff when
// M == N) are eligible.  Quantile: m_safe = margin, or +inf where the row is
// not eligible or the margin is NaN; thr = k_quant-th smallest m_safe over
// the B * M (row grain) or B * H * M (cell) entries, k_quant = max(1,
// int(q * n_elig)) from the host (0 when nothing is eligible); uncertain =
// m_safe <= thr and eligible.  Abs: uncertain = margin < tau and eligible.
// An uncertain cell keeps every visible block of its row.
// margin_eff: the head mean of each row for row grain (written for every
// head), a copy of the margins for cell grain; one thread per (b, row) or
// cell, over the whole grid.
__global__ __launch_bounds__(256) void router_rows_mean_kernel(
    const float* __restrict__ margin, int B, int H, int M, int grain,
    float* __restrict__ margin_eff) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (grain == kGrainRow) {
    if (i >= static_cast<int64_t>(B) * M) return;
    const int64_t b = i / M, row = i % M;
    const float mean = head_sum_in_order(margin + (b * H) * M + row, H, M) / static_cast<float>(H);
    for (int h = 0; h < H; ++h) margin_eff[(b * H + h) * M + row] = mean;
  } else {
    if (i >= static_cast<int64_t>(B) * H * M) return;
    margin_eff[i] = margin[i];
  }
}

__global__ __launch_bounds__(1024) void router_rows_threshold_kernel(
    int B, int H, int M, int grain, int rmode, int64_t k_quant, int elig_row0,
    const float* __restrict__ margin_eff, float* __restrict__ threshold) {
  __shared__ uint32_t hist[256 * kRouterWaves];
  __shared__ uint32_t s_prefix, s_remaining;
  const int tid = threadIdx.x;
  const int64_t n_all = static_cast<int64_t>(B) * H * M;
  if (rmode != kRouterQuantile || k_quant < 1) {
    if (tid == 0 && threshold != nullptr) *threshold = __uint_as_float(0x7FC00000u);
    return;
  }
  const int64_t n = grain == kGrainRow ? static_cast<int64_t>(B) * M : n_all;
  auto m_safe = [&](int64_t i) -> float {
    int64_t row, at;
    if (grain == kGrainRow) {
      row = i % M;
      at = ((i / M) * H) * M + row;
    } else {
      row = i % M;
      at = i;
    }
    const float e = margin_eff[at];
    return (row >= elig_row0 && e == e) ? e : INFINITY;
  };
  const float thr = key_float(block_kth_smallest(m_safe, n, k_quant, hist, &s_prefix, &s_remaining));
  if (tid == 0 && threshold != nullptr) *threshold = thr;
}

// Trigger decisions for 64 consecutive (b, h, row) cells per wavefront, one
// cell per lane (coalesced flag writes); then the wavefront writes the keep
// row of each triggered cell in turn: its visible blocks 0 .. row / 64.
__global__ __launch_bounds__(256) void router_rows_fill_kernel(
    const float* __restrict__ margin_eff, const float* __restrict__ threshold, int B, int H,
    int M, int NB, int rmode, float tau, int64_t k_quant, int elig_row0,
    uint8_t* __restrict__ uncertain, uint8_t* __restrict__ keep) {
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(B) * H * M;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 64;
  if (c0 >= n) return;
  const int64_t i = c0 + lane;
  bool unc = false;
  if (i < n) {
    const int row = static_cast<int>(i % M);
    const bool elig = row >= elig_row0;
    const float e = margin_eff[i];
    if (rmode == kRouterQuantile) {
      const float ms = e == e ? e : INFINITY;
      unc = k_quant > 0 && elig && ms <= *threshold;
    } else {
      unc = elig && e < tau;
    }
    uncertain[i] = unc ? 1 : 0;
  }
  const bool wide = (NB & 7) == 0 && (reinterpret_cast<uintptr_t>(keep) & 7) == 0;
  uint64_t pending = __ballot(unc);
  while (pending) {
    const int j = __ffsll(static_cast<long long>(pending)) - 1;
    pending &= pending - 1;
    const int64_t cell = c0 + j;
    uint8_t* kr = keep + cell * NB;
    const int last = static_cast<int>(cell % M) / kBlock;
    if (wide) {
      for (int b0 = 8 * lane; b0 < NB; b0 += 512) {   // eight flags per 8-byte store
        uint64_t w = 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) w |= static_cast<uint64_t>(b0 + q <= last) << (8 * q);
        *reinterpret_cast<uint64_t*>(kr + b0) = w;
      }
    } else {
      for (int blk = lane; blk < NB; blk += 64) kr[blk] = blk <= last ? 1 : 0;
    }
  }
}

hipError_t launch_router_rows(const float* margin, int B, int H, int M, int NB, int grain,
                              int rmode, float tau, int64_t k_quant, int elig_row0,
                              uint8_t* keep, float* margin_eff, uint8_t* uncertain,
                              float* threshold, hipStream_t stream) {
  const int64_t n_mean = grain == kGrainRow ? static_cast<int64_t>(B) * M
                                            : static_cast<int64_t>(B) * H * M;
  router_rows_mean_kernel<<<dim3(static_cast<unsigned>((n_mean + 255) / 256)), 256, 0, stream>>>(
      margin, B, H, M, grain, margin_eff);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  router_rows_threshold_kernel<<<1, 1024, 0, stream>>>(B, H, M, grain, rmode, k_quant, elig_row0,
                                                       margin_eff, threshold);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = static_cast<int64_t>(B) * H * M;
  const int64_t waves = (rows + 63) / 64;
  router_rows_fill_kernel<<<dim3(static_cast<unsigned>((waves + 3) / 4)), 256, 0, stream>>>(
      margin_eff, threshold, B, H, M, NB, rmode, tau, k_quant, elig_row0, uncertain, keep);
  return hipGetLastError();
}

}  // namespace ugbsa
