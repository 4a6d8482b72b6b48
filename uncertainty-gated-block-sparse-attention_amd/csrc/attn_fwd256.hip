// Kernel 3 at head_dim 256: the pipelined attention kernel (attn_pipe.h),
// one wavefront per 64-row tile, with the tile's O^T (256 registers) in the
// AGPR file, accumulated there by the P.V MFMAs; Q staged in LDS, one K / V^T
// register set.  (Two 32-row wavefronts per tile, each holding half of O^T
// in VGPRs, fetch every K / V^T block twice: 6-7 % slower at c5.)
#include "attn_pipe.h"

namespace ugbsa {

hipError_t launch_attn_pipe256(int elem, const uint16_t* q, int64_t sq_b, int64_t sq_h,
                               int64_t sq_m, const uint16_t* k, int64_t sk_b, int64_t sk_h,
                               int64_t sk_n, const uint16_t* vt, const int32_t* kv_idx,
                               const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                               int64_t si_t, int B, int H, int Hk, int M, int N, int Qt,
                               int k_slots, float scale, uint16_t* out, int64_t so_b,
                               int64_t so_h, int64_t so_m, hipStream_t stream,
                               const int32_t* tile_order) {
  if (elem == ElemF16::code)
    return launch_attn_pipe<ElemF16, 256, 4, true, true, true>(
        q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, H, Hk,
        M, N, Qt, k_slots, scale, out, so_b, so_h, so_m, stream, tile_order);
  return launch_attn_pipe<ElemBf16, 256, 4, true, true, true>(
      q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, H, Hk, M,
      N, Qt, k_slots, scale, out, so_b, so_h, so_m, stream, tile_order);
}

}  // namespace ugbsa
