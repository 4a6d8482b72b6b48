// Kernel 3 at head_dim 128 for long contexts: the pipelined attention
// kernel (attn_pipe.h) with one K / V^T register set per wavefront, each
// requested one phase ahead of use, instead of two sets requested two half
// blocks ahead.  With 128K-token contexts (2048 K blocks per head) the
// gathered blocks mostly miss L2, and the deeper prefetch keeps as many bytes
// in flight per XCD as its L2 holds (128 wavefronts x 32 KiB = 4 MiB); the
// shallower one halves that and keeps more of the blocks shared between the
// query heads of a KV group resident.  Measured on MI355X: 7-10 % faster
// than the deep prefetch at 128K, 5 % slower at 64K and 3 % at 32K, hence
// launch_attn_fwd's switch at 1024 blocks.
#include "attn_pipe.h"

namespace ugbsa {

hipError_t launch_attn_pipe128_long(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                    const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                    const uint16_t* vt, const int32_t* kv_idx,
                                    const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                                    int64_t si_t, int B, int H, int Hk, int M, int N, int Qt,
                                    int k_slots, float scale, uint16_t* out, int64_t so_b,
                                    int64_t so_h, int64_t so_m, hipStream_t stream,
                                    const int32_t* tile_order) {
  return launch_attn_pipe<128, 4, false, true>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt,
                                               kv_idx, rowmask, si_b, si_h, si_t, B, H, Hk, M,
                                               N, Qt, k_slots, scale, out, so_b, so_h, so_m,
                                               stream, tile_order);
}

}  // namespace ugbsa
