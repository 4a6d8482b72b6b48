// Kernel 2 compile unit: the bf16 selection kernels (select.h), the v1
// per-row selector and the element-format dispatch.
#include "select.h"

namespace ugbsa {

// v1 per-row selection (src/sparse_attention.py:245-295, 299-325 for the
// margin): one wavefront per query row.  The row's visible scores (blocks
// 0 .. row / 64, M == N) are ranked K deep by the same radix select and
// bitonic sort as the tile selector; the kept blocks are the count best —
// count = k_bud, or for belief clamp(#{j : cumsum_j < top_p} + 1, k_min,
// k_max) over the sorted softmax probabilities — then ranks past the
// visible blocks take the lowest invisible blocks (the total order's -inf
// ties), and the sink and the row's own block are forced.  The keep row is
// assembled as flags in the wave's LDS row and written once.
__host__ __device__ constexpr int rows_wave_bytes(int NB, int KP) {
  return (NB * 4 + 15) / 16 * 16 + 256 * 4 + KP * 8;
}

template <int KP, int RK>
__global__ __launch_bounds__(256) void select_rows_kernel(const RowsArgs a) {
  constexpr int R = KP / 64;
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (gid >= static_cast<int64_t>(a.B) * a.H * a.nrows) return;
  const int64_t bh = gid / a.nrows;
  const int row = a.r0 + static_cast<int>(gid % a.nrows);
  if (row >= a.M) return;
  const int h = static_cast<int>(bh % a.H);
  const int NB = a.NB;
  unsigned char* wreg = smem + wave * rows_wave_bytes(NB, KP);
  float* trow = reinterpret_cast<float*>(wreg);
  uint32_t* hist = reinterpret_cast<uint32_t*>(wreg + (NB * 4 + 15) / 16 * 16);
  uint64_t* cand = reinterpret_cast<uint64_t*>(wreg + (NB * 4 + 15) / 16 * 16 + 1024);
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));

  const int n_vis = row / kBlock + 1;
  const float* src = a.scores + gid * NB;
  const bool pen = a.penalty != nullptr && row == a.M - 1;
  for (int blk = lane; blk < n_vis; blk += 64)
    trow[blk] = pen ? src[blk] - a.penalty[static_cast<int64_t>(h) * NB + blk] : src[blk];
  wave_lds_sync();

  const int K = a.K;
  select_to_cand<RK>(trow, n_vis, K, hist, cand, lane, lt_mask);
  wave_lds_sync();
  const int n_sel = min(n_vis, K);
  uint64_t v[R];
  sort_cand<KP>(cand, n_sel, lane, v);

  int count = a.k_bud;
  if (a.belief) {
    // softmax over the visible blocks (max-subtracted, fp32), then the
    // cumulative mass of the sorted probabilities
    const float mx = sorted_value<R>(v, 0, n_sel);
    float z = 0.f;
    for (int blk = lane; blk < n_vis; blk += 64) z += expf(trow[blk] - mx);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) z += shfl_xor_f(z, m);
    float carry = 0.f;
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = lane + 64 * r;
      float c = e < n_sel ? expf(key_float(static_cast<uint32_t>(v[r] >> 32)) - mx) / z : 0.f;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float o = __shfl_up(c, d, 64);
        if (lane >= d) c += o;
      }
      c += carry;
      carry = __shfl(c, 63, 64);
      cnt += __popcll(__ballot(e < K && c < a.top_p));
    }
    count = cnt + 1;
    if (count < a.k_min) count = a.k_min;
    if (count > a.k_max) count = a.k_max;
  }

  // keep flags in the LDS row (its scores are no longer needed)
  uint32_t* flag = reinterpret_cast<uint32_t*>(trow);
  wave_lds_sync();
  for (int blk = lane; blk < NB; blk += 64) flag[blk] = 0u;
  wave_lds_sync();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int e = lane + 64 * r;
    if (e < n_sel && e < count) flag[0xFFFFFFFFu - static_cast<uint32_t>(v[r])] = 1u;
  }
  for (int blk = n_vis + lane; blk < min(count, NB); blk += 64) flag[blk] = 1u;
  if (lane == 0) {
    flag[0] = 1u;
    flag[row / kBlock] = 1u;
  }
  wave_lds_sync();
  uint8_t* kr = a.keep + (bh * a.M + row) * NB;
  if ((NB & 7) == 0 && (reinterpret_cast<uintptr_t>(a.keep) & 7) == 0) {
    // eight flags per lane packed into one 8-byte store
    for (int b0 = 8 * lane; b0 < NB; b0 += 512) {
      uint64_t w = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) w |= static_cast<uint64_t>(flag[b0 + i] & 1u) << (8 * i);
      *reinterpret_cast<uint64_t*>(kr + b0) = w;
    }
  } else {
    for (int blk = lane; blk < NB; blk += 64) kr[blk] = static_cast<uint8_t>(flag[blk]);
  }

  if (a.margin != nullptr) {
    // (s[k_eff - 1] - s[k_eff]) / max(s[0] - s[k_eff], 1e-6); NaN kept
    const float s_top = sorted_value<R>(v, 0, n_sel);
    const float s_km1 = sorted_value<R>(v, a.k_eff - 1, n_sel);
    const float s_k = sorted_value<R>(v, a.k_eff, n_sel);
    float spread = s_top - s_k;
    if (spread < 1e-6f) spread = 1e-6f;
    const float mg = (s_km1 - s_k) / spread;
    if (lane == 0) a.margin[bh * a.M + row] = mg;
  }
}

template <int KP, int RK>
static hipError_t launch_rows_t(const RowsArgs& a, hipStream_t stream) {
  const size_t lds = 4 * static_cast<size_t>(rows_wave_bytes(a.NB, KP));
  if (lds > 160 * 1024) return hipErrorInvalidConfiguration;
  auto kern = select_rows_kernel<KP, RK>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds));
  if (e != hipSuccess) return e;
  const int64_t waves = static_cast<int64_t>(a.B) * a.H * a.nrows;
  kern<<<dim3(static_cast<unsigned>((waves + 3) / 4)), 256, lds, stream>>>(a);
  return hipGetLastError();
}

// Keys held in registers per lane: the row's blocks / 64, so that short rows
// keep fewer registers live and more wavefronts fit on a SIMD (this kernel
// is latency-bound: one row per wavefront).
template <int KP>
static hipError_t launch_rows_k(const RowsArgs& a, hipStream_t stream) {
  if (a.NB <= 64 * 8) return launch_rows_t<KP, 8>(a, stream);
  if (a.NB <= 64 * 16) return launch_rows_t<KP, 16>(a, stream);
  return launch_rows_t<KP, kRegKeys>(a, stream);
}

hipError_t launch_select_rows(const RowsArgs& a, hipStream_t stream) {
  if (a.K <= 64) return launch_rows_k<64>(a, stream);
  if (a.K <= 128) return launch_rows_k<128>(a, stream);
  if (a.K <= 256) return launch_rows_k<256>(a, stream);
  if (a.K <= 512) return launch_rows_k<512>(a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_select(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                         const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                         int elem, int mode, float scaling, int k_base, int k_slots,
                         int want_sigma, int32_t* kv_idx, float* sigma, float* tile_score,
                         hipStream_t stream, const SelectAux* aux) {
  if (elem == ElemF16::code)
    return launch_select_f16(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, D, mode, scaling,
                             k_base, k_slots, want_sigma, kv_idx, sigma, tile_score, stream, aux);
  return launch_select_e<ElemBf16>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, D, mode, scaling,
                                   k_base, k_slots, want_sigma, kv_idx, sigma, tile_score, stream,
                                   aux);
}

}  // namespace ugbsa
