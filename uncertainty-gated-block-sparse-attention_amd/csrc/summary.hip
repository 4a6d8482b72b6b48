// Kernel 1: per-block K summaries for block scoring (HBM-bound, K read once).
//
// Restates src/sparse_attention.py:618-622, 636-637, 646 of the reference on
// the GQA key tensor [B, Hk, N, D] (the reference works on the repeat_kv'd
// copy; the summaries of repeated heads are identical).  Rows past N count as
// zeros, as F.pad does for the last partial block.
//
// Output "planes" [B, Hk, NB, P, D] in K's 16-bit format (bf16 or fp16) is
// the operand layout of the scoring kernel: P = 2 for Quest (K-max, K-min —
// input values, exact) and P = 3 for the mean, stored as an unevaluated sum
// hi + mid + lo of three 16-bit values, so the MFMA contraction
// q . (hi + mid + lo) follows an fp32 q . mean: in bf16 to within an fp32
// rounding of the mean; in fp16 the lo term can fall in fp16's subnormal
// range, which bounds the error of the sum by 2^-25 absolute (against
// 2^-24 relative for an fp32 mean).
#include "common.h"
#include "launch.h"

namespace ugbsa {

template <int D, typename E>
__global__ __launch_bounds__(256) void block_summary_kernel(
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    int Hk, int N, int NB, int mode, uint16_t* __restrict__ planes) {
  constexpr int CH = D / 8;        // 16-byte chunks per row
  constexpr int RG = 256 / CH;     // row groups
  constexpr int RPG = kBlock / RG; // rows per group
  __shared__ float red[3][RG][D + 1];

  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int c = threadIdx.x % CH, rg = threadIdx.x / CH;
  const uint16_t* base = k + b * sk_b + h * sk_h + static_cast<int64_t>(c) * 8;

  float s[8], mn[8], mx[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) { s[j] = 0.f; mn[j] = INFINITY; mx[j] = -INFINITY; }

#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    const int row = blk * kBlock + r * RG + rg;
    u32x4 raw = {0u, 0u, 0u, 0u};
    if (row < N) raw = *reinterpret_cast<const u32x4*>(base + row * sk_n);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = E::to_f32(raw[j] & 0xFFFFu);
      const float hi = E::to_f32(raw[j] >> 16);
      s[2 * j] += lo; s[2 * j + 1] += hi;
      mn[2 * j] = fminf(mn[2 * j], lo); mn[2 * j + 1] = fminf(mn[2 * j + 1], hi);
      mx[2 * j] = fmaxf(mx[2 * j], lo); mx[2 * j + 1] = fmaxf(mx[2 * j + 1], hi);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    red[0][rg][c * 8 + j] = s[j];
    red[1][rg][c * 8 + j] = mn[j];
    red[2][rg][c * 8 + j] = mx[j];
  }
  __syncthreads();

  const int P = mode == kModeQuest ? 2 : 3;
  uint16_t* out = planes + ((static_cast<int64_t>(b) * Hk + h) * NB + blk) * P * D;
  for (int d = threadIdx.x; d < D; d += 256) {
    if (mode == kModeQuest) {
      float a = -INFINITY, z = INFINITY;
      for (int g = 0; g < RG; ++g) { a = fmaxf(a, red[2][g][d]); z = fminf(z, red[1][g][d]); }
      out[d] = E::from_f32(a);          // exact: an input value (or 0)
      out[D + d] = E::from_f32(z);
    } else {
      float acc = 0.f;
      for (int g = 0; g < RG; ++g) acc += red[0][g][d];
      const float mean = acc * (1.0f / kBlock);
      const uint16_t h0 = E::from_f32(mean);
      const float r1 = mean - E::to_f32(h0);
      const uint16_t h1 = E::from_f32(r1);
      const float r2 = r1 - E::to_f32(h1);
      out[d] = h0;
      out[D + d] = h1;
      out[2 * D + d] = E::from_f32(r2);
    }
  }
}

template <typename E>
static hipError_t launch_block_summary_e(const uint16_t* k, int64_t sk_b, int64_t sk_h,
                                         int64_t sk_n, int B, int Hk, int N, int D, int mode,
                                         uint16_t* planes, hipStream_t stream) {
  const int NB = (N + kBlock - 1) / kBlock;
  dim3 grid(NB, Hk, B);
  switch (D) {
    case 64:
      block_summary_kernel<64, E><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, Hk, N, NB, mode, planes);
      break;
    case 128:
      block_summary_kernel<128, E><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, Hk, N, NB, mode, planes);
      break;
    case 256:
      block_summary_kernel<256, E><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, Hk, N, NB, mode, planes);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_block_summary(const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                int B, int Hk, int N, int D, int elem, int mode,
                                uint16_t* planes, hipStream_t stream) {
  if (elem == ElemF16::code)
    return launch_block_summary_e<ElemF16>(k, sk_b, sk_h, sk_n, B, Hk, N, D, mode, planes, stream);
  return launch_block_summary_e<ElemBf16>(k, sk_b, sk_h, sk_n, B, Hk, N, D, mode, planes, stream);
}

}  // namespace ugbsa
