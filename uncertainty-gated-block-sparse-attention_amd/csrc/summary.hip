// Kernel 1: per-block K summaries for block scoring (HBM-bound, K read once).
//
// Restates src/sparse_attention.py:618-622, 636-637, 646 of the reference on
// the GQA key tensor [B, Hk, N, D] (the reference works on the repeat_kv'd
// copy; the summaries of repeated heads are identical).  Rows past N count as
// zeros, as F.pad does for the last partial block.
//
// Output "planes", the operand layout of the scoring kernel:
//  * Quest: [B, Hk, NB, 2, D] in K's 16-bit format (bf16 or fp16): K-max,
//    K-min — input values, exact.
//  * mean, for both formats: [B, Hk, NB, 2, D] fp16, then [B, Hk, NB] fp32.
//    The fp32 mean m of a block is scaled by 2^e, e = 141 - (the fp32
//    exponent field of max_d |m_d|), so that max_d |m_d| 2^e lies in
//    [2^14, 2^15), and stored as the unevaluated sum hi + lo of two fp16
//    values (hi = fp16(m 2^e), lo = fp16(m 2^e - hi)); the fp32 array holds
//    2^-e.  hi + lo carries 22-23 significant bits of each m_d 2^e: the sum
//    is within 2^-23 |m_d| 2^e + 2^-25 of it (the second term where lo falls
//    in fp16's subnormal range, i.e. 2^-39 of the block's largest |m_d|).
//    The scoring kernel multiplies fp16 Q (scaled by a power of two per
//    tile, exact) by both planes on the fp16 MFMA — two contractions per
//    block instead of the three that a bf16 hi + mid + lo split of the fp32
//    mean takes — and undoes both scales exactly on the fp32 result.
#include "common.h"
#include "launch.h"

namespace ugbsa {

template <int D, typename E>
__global__ __launch_bounds__(256) void block_summary_kernel(
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    int B, int Hk, int N, int NB, int mode, uint16_t* __restrict__ planes) {
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

  if (mode == kModeQuest) {
    uint16_t* out = planes + ((static_cast<int64_t>(b) * Hk + h) * NB + blk) * 2 * D;
    for (int d = threadIdx.x; d < D; d += 256) {
      float a = -INFINITY, z = INFINITY;
      for (int g = 0; g < RG; ++g) { a = fmaxf(a, red[2][g][d]); z = fminf(z, red[1][g][d]); }
      out[d] = E::from_f32(a);          // exact: an input value (or 0)
      out[D + d] = E::from_f32(z);
    }
    return;
  }
  // mean: one d per thread (D <= 256 threads), the block's largest |mean|
  // over d through LDS, then the scaled two-term fp16 split
  __shared__ uint32_t wmax[4];
  const int d = threadIdx.x;
  float mean = 0.f;
  if (d < D) {
    float acc = 0.f;
    for (int g = 0; g < RG; ++g) acc += red[0][g][d];
    mean = acc * (1.0f / kBlock);
  }
  uint32_t mb = __float_as_uint(mean) & 0x7FFFFFFFu;     // |mean| orders as its bits
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mb = max(mb, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mb), m, 64)));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mb;
  __syncthreads();
  const uint32_t bmax = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
  const int e = bmax == 0u ? 0 : 141 - static_cast<int>(bmax >> 23);
  const int64_t bid = (static_cast<int64_t>(b) * Hk + h) * NB + blk;
  if (d < D) {
    uint16_t* out = planes + bid * 2 * D;
    const float x = ldexpf(mean, e);                   // exact
    const uint16_t hi = ElemF16::from_f32(x);
    out[d] = hi;
    out[D + d] = ElemF16::from_f32(x - ElemF16::to_f32(hi));
  }
  if (threadIdx.x == 0) {
    float* descale = reinterpret_cast<float*>(planes + static_cast<int64_t>(B) * Hk * NB * 2 * D);
    descale[bid] = ldexpf(1.0f, -e);
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
      block_summary_kernel<64, E><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, B, Hk, N, NB, mode, planes);
      break;
    case 128:
      block_summary_kernel<128, E><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, B, Hk, N, NB, mode, planes);
      break;
    case 256:
      block_summary_kernel<256, E><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, B, Hk, N, NB, mode, planes);
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
