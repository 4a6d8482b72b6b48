// Kernel 2 compile unit: the fp16 instances of the selection kernels
// (select.h), compiled apart from the bf16 ones so that both build in
// parallel.
#include "select.h"

namespace ugbsa {

hipError_t launch_select_f16(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                             const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                             int mode, float scaling, int k_base, int k_slots, int want_sigma,
                             int32_t* kv_idx, float* sigma, float* tile_score,
                             hipStream_t stream, const SelectAux* aux) {
  return launch_select_e<ElemF16>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, D, mode, scaling,
                                  k_base, k_slots, want_sigma, kv_idx, sigma, tile_score, stream,
                                  aux);
}

}  // namespace ugbsa
