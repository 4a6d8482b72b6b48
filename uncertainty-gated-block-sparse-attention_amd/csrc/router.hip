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
// workgroup (an 8-bit radix select, 4 passes over <= B * H * Qt values that
// sit in L2), followed by a grid-wide fill.
#include "common.h"
#include "launch.h"

namespace ugbsa {

__global__ __launch_bounds__(1024) void router_threshold_kernel(
    const float* __restrict__ sigma, int B, int H, int Qt, int grain, int rmode, float tau,
    int64_t k_quant, float* __restrict__ sigma_eff, uint8_t* __restrict__ uncertain,
    float* __restrict__ threshold) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_remaining;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t n_all = static_cast<int64_t>(B) * H * Qt;

  // 1. effective sigma
  if (grain == kGrainRow) {
    for (int64_t i = tid; i < static_cast<int64_t>(B) * Qt; i += nt) {
      const int b = static_cast<int>(i / Qt), t = static_cast<int>(i % Qt);
      float acc = sigma[(static_cast<int64_t>(b) * H) * Qt + t];
      for (int h = 1; h < H; ++h) acc = acc + sigma[(static_cast<int64_t>(b) * H + h) * Qt + t];
      const float mean = acc / static_cast<float>(H);
      for (int h = 0; h < H; ++h) sigma_eff[(static_cast<int64_t>(b) * H + h) * Qt + t] = mean;
    }
  } else {
    for (int64_t i = tid; i < n_all; i += nt) sigma_eff[i] = sigma[i];
  }
  __syncthreads();

  // 2. threshold
  float thr = tau;
  if (rmode == kRouterQuantile) {
    // rank among the values examined: per-tile means (row) or all cells
    const int64_t n = grain == kGrainRow ? static_cast<int64_t>(B) * Qt : n_all;
    const int64_t kth = grain == kGrainRow ? (k_quant - 1) / H + 1 : k_quant;  // 1-based
    auto value_at = [&](int64_t i) -> float {
      if (grain == kGrainRow) {
        const int64_t b = i / Qt, t = i % Qt;
        return sigma_eff[(b * H) * Qt + t];
      }
      return sigma_eff[i];
    };
    if (tid == 0) { s_prefix = 0; s_remaining = static_cast<uint32_t>(kth); }
    uint32_t pmask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += nt) hist[i] = 0;
      __syncthreads();
      const uint32_t prefix = s_prefix;
      for (int64_t i = tid; i < n; i += nt) {
        const uint32_t key = float_key(value_at(i));
        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {   // ascending scan for the bin holding the remaining-th smallest
        uint32_t rem = s_remaining, below = 0;
        for (int d = 0; d < 256; ++d) {
          if (below + hist[d] >= rem) {
            s_prefix = prefix | (static_cast<uint32_t>(d) << shift);
            s_remaining = rem - below;
            break;
          }
          below += hist[d];
        }
      }
      pmask |= 0xFFu << shift;
      __syncthreads();
    }
    thr = key_float(s_prefix);
  }
  if (tid == 0 && threshold != nullptr) *threshold = thr;

  // 3. decision (NaN never triggers: comparisons with NaN are false)
  for (int64_t i = tid; i < n_all; i += nt) {
    const float e = sigma_eff[i];
    uncertain[i] = rmode == kRouterQuantile ? (e <= thr) : (e < tau);
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
  router_threshold_kernel<<<1, 1024, 0, stream>>>(sigma, B, H, Qt, grain, rmode, tau, k_quant,
                                                  sigma_eff, uncertain, threshold);
  hipError_t e = hipGetLastError();
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

}  // namespace ugbsa
