// extern "C" boundary of libugbsa: argument validation, error reporting,
// dispatch to the kernel launchers.  Declarations and the reference
// interfaces each entry point replaces: include/ugbsa.h.
#include <cstdio>
#include <cstdarg>
#include <mutex>
#include <string>

#include "common.h"
#include "launch.h"
#include "../../include/ugbsa.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_result(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_error.clear();
    return UGBSA_OK;
  }
  return fail(static_cast<int>(e), "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks a bf16 [B, H, S, D] operand read with 16-byte vector loads.
int check_bf16_operand(const char* name, const void* p, int64_t s_b, int64_t s_h, int64_t s_s,
                       int64_t s_d) {
  if (p == nullptr) return fail(UGBSA_EARG, "%s is null", name);
  if (s_d != 1) return fail(UGBSA_ELAYOUT, "%s: innermost (head_dim) stride must be 1, got %lld", name, (long long)s_d);
  if (!aligned16(p)) return fail(UGBSA_ELAYOUT, "%s: data pointer must be 16-byte aligned", name);
  if (s_b % 8 || s_h % 8 || s_s % 8)
    return fail(UGBSA_ELAYOUT, "%s: batch/head/sequence strides must be multiples of 8 elements", name);
  return UGBSA_OK;
}

int check_dims(int B, int H, int Hk, int D, int dtype) {
  if (dtype != UGBSA_DTYPE_BF16 && dtype != UGBSA_DTYPE_F16)
    return fail(UGBSA_EDTYPE, "only bf16 and fp16 tensors are supported (dtype code %d)", dtype);
  if (B < 1 || H < 1 || Hk < 1) return fail(UGBSA_EARG, "B, H, Hk must be positive");
  if (H % Hk) return fail(UGBSA_EARG, "query heads (%d) must be a multiple of key heads (%d)", H, Hk);
  if (D != 64 && D != 128 && D != 256) return fail(UGBSA_EARG, "head_dim %d not supported (64, 128, 256)", D);
  return UGBSA_OK;
}

// bf16 elements of the K and V operand copies in the attention workspace;
// the tile schedule (2 * B * NB int32: per-tile work, then the tile order)
// follows them.
int64_t kv_copy_elems(int B, int Hk, int N, int D) {
  const int64_t nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  return 2 * static_cast<int64_t>(B) * Hk * nb * ugbsa::kBlock * D;
}

}  // namespace

extern "C" {

int ugbsa_abi_version(void) { return UGBSA_ABI_VERSION; }

const char* ugbsa_last_error(void) { return g_error.c_str(); }

int64_t ugbsa_summary_elems(int B, int Hk, int N, int D, int mode) {
  const int64_t nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  // Quest: two planes in the call's format; mean: two fp16 planes, then one
  // fp32 scale (two 16-bit elements) per block
  return static_cast<int64_t>(B) * Hk * nb * (mode == UGBSA_MODE_QUEST ? 2 * D : 2 * D + 2);
}

int64_t ugbsa_attn_workspace_elems(int B, int Hk, int N, int D) {
  const int64_t nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  const int64_t sched = (4 * static_cast<int64_t>(B) * nb + 7) / 8 * 8;   // 2 B NB int32
  return kv_copy_elems(B, Hk, N, D) + sched;
}

int ugbsa_block_summary(const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                        int B, int Hk, int N, int D, int dtype, int mode, void* planes,
                        void* stream) {
  int rc = check_dims(B, Hk, Hk, D, dtype);
  if (rc) return rc;
  if ((rc = check_bf16_operand("k", k, sk_b, sk_h, sk_n, sk_d))) return rc;
  if (N < 1) return fail(UGBSA_EARG, "N must be positive");
  if (mode != UGBSA_MODE_MEAN && mode != UGBSA_MODE_QUEST) return fail(UGBSA_EARG, "unknown score mode %d", mode);
  if (planes == nullptr) return fail(UGBSA_EARG, "planes is null");
  // the mean's fp32 block scales follow the planes; the selection reads
  // the planes with 16-byte loads
  if (!aligned16(planes)) return fail(UGBSA_ELAYOUT, "planes must be 16-byte aligned");
  return hip_result(ugbsa::launch_block_summary(static_cast<const uint16_t*>(k), sk_b, sk_h, sk_n, B, Hk, N, D,
                                                dtype, mode, static_cast<uint16_t*>(planes),
                                                static_cast<hipStream_t>(stream)),
                    "block_summary");
}

int ugbsa_select(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                 const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                 int mode, float scaling, int k_base, int k_slots, int block_m, int32_t* kv_idx,
                 float* sigma, float* tile_score, void* stream) {
  int rc = check_dims(B, H, Hk, D, dtype);
  if (rc) return rc;
  if ((rc = check_bf16_operand("q", q, sq_b, sq_h, sq_m, sq_d))) return rc;
  if (M < 1 || N < 1) return fail(UGBSA_EARG, "M and N must be positive");
  // tile visibility takes query row i as key position i (one-shot prefill)
  if (M != N) return fail(UGBSA_EARG, "selection needs query length == key length (M=%d, N=%d)", M, N);
  if (block_m != 64) return fail(UGBSA_EARG, "selection tiles are 64 rows (block_m=%d)", block_m);
  if (mode != UGBSA_MODE_MEAN && mode != UGBSA_MODE_QUEST) return fail(UGBSA_EARG, "unknown score mode %d", mode);
  if (planes == nullptr || kv_idx == nullptr) return fail(UGBSA_EARG, "planes / kv_idx is null");
  if (!aligned16(planes)) return fail(UGBSA_ELAYOUT, "planes must be 16-byte aligned");
  const int nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  if (nb > ugbsa::kMaxBlocksSelect) return fail(UGBSA_EARG, "N=%d gives %d key blocks; the selector holds at most %d", N, nb, ugbsa::kMaxBlocksSelect);
  if (k_slots < 1 || k_slots > nb || k_slots > ugbsa::kMaxSlots)
    return fail(UGBSA_EARG, "k_slots=%d out of range [1, min(NB=%d, %d)]", k_slots, nb, ugbsa::kMaxSlots);
  if (k_base < 1 || k_base > k_slots) return fail(UGBSA_EARG, "k_base=%d out of range [1, k_slots=%d]", k_base, k_slots);
  if (sigma != nullptr && k_base >= k_slots) return fail(UGBSA_EARG, "sigma needs k_base < k_slots");
  return hip_result(ugbsa::launch_select(static_cast<const uint16_t*>(q), sq_b, sq_h, sq_m,
                                         static_cast<const uint16_t*>(planes), B, H, Hk, M, N, D,
                                         dtype, mode, scaling, k_base, k_slots, sigma != nullptr, kv_idx,
                                         sigma, tile_score, static_cast<hipStream_t>(stream)),
                    "select");
}

int ugbsa_score_dump(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                     const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                     int mode, float scaling, int k_b, int rho_k, float* g, float* r,
                     float* sigma, float* g_rho, uint8_t* valid, float* tau_hat,
                     float* tile_score, void* stream) {
  int rc = check_dims(B, H, Hk, D, dtype);
  if (rc) return rc;
  if ((rc = check_bf16_operand("q", q, sq_b, sq_h, sq_m, sq_d))) return rc;
  if (M < 1 || N < 1) return fail(UGBSA_EARG, "M and N must be positive");
  if (mode != UGBSA_MODE_MEAN && mode != UGBSA_MODE_QUEST) return fail(UGBSA_EARG, "unknown score mode %d", mode);
  if (planes == nullptr) return fail(UGBSA_EARG, "planes is null");
  if (!aligned16(planes)) return fail(UGBSA_ELAYOUT, "planes must be 16-byte aligned");
  if (g == nullptr || r == nullptr || sigma == nullptr || g_rho == nullptr || valid == nullptr ||
      tau_hat == nullptr)
    return fail(UGBSA_EARG, "g / r / sigma / g_rho / valid / tau_hat is null");
  const int nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  if (nb > ugbsa::kMaxBlocksSelect) return fail(UGBSA_EARG, "N=%d gives %d key blocks; the selector holds at most %d", N, nb, ugbsa::kMaxBlocksSelect);
  if (k_b < 1 || k_b >= rho_k || rho_k >= nb || rho_k + 1 > ugbsa::kMaxSlots)
    return fail(UGBSA_EARG, "score dump needs 1 <= k_b < rho_k < min(NB=%d, %d) (k_b=%d, rho_k=%d)",
                nb, ugbsa::kMaxSlots, k_b, rho_k);
  hipStream_t st = static_cast<hipStream_t>(stream);
  ugbsa::SelectAux dump;
  dump.g = g;
  dump.r = r;
  dump.sigma = sigma;
  dump.g_rho = g_rho;
  dump.valid = valid;
  dump.k_b = k_b;
  dump.rho_k = rho_k;
  dump.dump = 1;
  const uint16_t* q16 = static_cast<const uint16_t*>(q);
  const uint16_t* p16 = static_cast<const uint16_t*>(planes);
  hipError_t e = ugbsa::launch_select(q16, sq_b, sq_h, sq_m, p16, B, H, Hk, M, N, D, dtype, mode, scaling,
                                      k_b, rho_k + 1, 0, nullptr, nullptr, tile_score, st, &dump);
  if (e != hipSuccess) return hip_result(e, "score_dump select");
  return hip_result(ugbsa::launch_score_tau(q16, sq_b, sq_h, sq_m, p16, B, H, Hk, M, N, D, dtype, mode,
                                            scaling, tau_hat, st),
                    "score_dump tau");
}

int ugbsa_router(const float* sigma, int B, int H, int Qt, int grain, int rmode, float tau,
                 int64_t k_quant, int32_t* kv_idx, int k_base, int k_slots, int NB,
                 float* sigma_eff, uint8_t* uncertain, float* threshold, void* stream) {
  if (sigma == nullptr || kv_idx == nullptr || sigma_eff == nullptr || uncertain == nullptr)
    return fail(UGBSA_EARG, "sigma / kv_idx / sigma_eff / uncertain is null");
  if (B < 1 || H < 1 || Qt < 1) return fail(UGBSA_EARG, "B, H, Qt must be positive");
  if (grain != UGBSA_GRAIN_CELL && grain != UGBSA_GRAIN_ROW) return fail(UGBSA_EARG, "unknown router grain %d", grain);
  if (rmode != UGBSA_ROUTER_ABS && rmode != UGBSA_ROUTER_QUANTILE) return fail(UGBSA_EARG, "unknown router mode %d", rmode);
  const int64_t n = static_cast<int64_t>(B) * H * Qt;
  if (rmode == UGBSA_ROUTER_QUANTILE && (k_quant < 1 || k_quant > n))
    return fail(UGBSA_EARG, "k_quant=%lld out of range [1, %lld]", (long long)k_quant, (long long)n);
  if (k_base < 1 || k_base >= k_slots || k_slots > NB)
    return fail(UGBSA_EARG, "router needs 1 <= k_base < k_slots <= NB (%d, %d, %d)", k_base, k_slots, NB);
  return hip_result(ugbsa::launch_router(sigma, B, H, Qt, grain, rmode, tau, k_quant, kv_idx, k_base,
                                         k_slots, NB, sigma_eff, uncertain, threshold,
                                         static_cast<hipStream_t>(stream)),
                    "router");
}

int ugbsa_attn_prepare_kv(const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                          const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                          int B, int Hk, int N, int D, int dtype, int block_m, void* workspace,
                          int64_t workspace_elems, void* stream) {
  int rc = check_dims(B, Hk, Hk, D, dtype);
  if (rc) return rc;
  if ((rc = check_bf16_operand("k", k, sk_b, sk_h, sk_n, sk_d))) return rc;
  if ((rc = check_bf16_operand("v", v, sv_b, sv_h, sv_n, sv_d))) return rc;
  if (N < 1) return fail(UGBSA_EARG, "N must be positive");
  if (block_m != 64 && block_m != 32) return fail(UGBSA_EARG, "block_m must be 64 or 32 (got %d)", block_m);
  if (workspace == nullptr || !aligned16(workspace)) return fail(UGBSA_EARG, "workspace must be a 16-byte aligned buffer");
  if (workspace_elems < kv_copy_elems(B, Hk, N, D))
    return fail(UGBSA_EARG, "workspace of %lld elements holds less than the K/V operand copies (%lld)",
                (long long)workspace_elems, (long long)kv_copy_elems(B, Hk, N, D));
  if (kv_copy_elems(1, 1, N, D) * 2 > 0xFFFFFFFFLL)
    return fail(UGBSA_EARG, "one KV head's K/V copy exceeds 4 GiB (N=%d, D=%d)", N, D);
  return hip_result(ugbsa::launch_attn_prepare(static_cast<const uint16_t*>(k), sk_b, sk_h, sk_n,
                                               static_cast<const uint16_t*>(v), sv_b, sv_h, sv_n,
                                               B, Hk, N, D, block_m,
                                               static_cast<uint16_t*>(workspace),
                                               static_cast<hipStream_t>(stream)),
                    "attn_prepare_kv");
}

}  // extern "C"

namespace {

// ---- static scratch of ugbsa_select_mask_static ---------------------------
// The per-row scores of the v1 selector's passes live in this file-scope
// array instead of a caller workspace: kStaticScratchFloats fp32 (64 MiB) on
// every device the library runs on, held until the process ends.  Host code
// must not pass the array's name to a kernel (it is a host-side stand-in);
// its device address is looked up once per device, with that device current,
// and kept in g_scratch_ptr.
constexpr int64_t kStaticScratchFloats = int64_t(1) << 24;
constexpr int kMaxDevices = 64;
__device__ __align__(256) float scratch[kStaticScratchFloats];
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

int static_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_result(e, "select_mask_static: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(UGBSA_EARG, "device %d beyond the %d the static scratch tracks", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_result(e, "select_mask_static: hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(UGBSA_EARG, "select_mask_static: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<float*>(g_scratch_ptr[dev]);
  return UGBSA_OK;
}

int select_mask_impl(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                      const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                      int mode, float scaling, int policy, int k_bud, int k_eff, int k_min,
                      int k_max, float top_p, const float* penalty, float* workspace,
                      int64_t workspace_elems, uint8_t* keep, float* margin, void* stream) {
  int rc = check_dims(B, H, Hk, D, dtype);
  if (rc) return rc;
  if ((rc = check_bf16_operand("q", q, sq_b, sq_h, sq_m, sq_d))) return rc;
  if (M < 1 || M != N) return fail(UGBSA_EARG, "the per-row selector needs M == N >= 1 (M=%d, N=%d)", M, N);
  if (mode != UGBSA_MODE_MEAN && mode != UGBSA_MODE_QUEST) return fail(UGBSA_EARG, "unknown score mode %d", mode);
  if (policy != UGBSA_V1_TOPK && policy != UGBSA_V1_BELIEF) return fail(UGBSA_EARG, "unknown v1 policy %d", policy);
  if (planes == nullptr || !aligned16(planes)) return fail(UGBSA_ELAYOUT, "planes must be a 16-byte aligned buffer");
  if (keep == nullptr) return fail(UGBSA_EARG, "keep is null");
  const int nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  if (nb > ugbsa::kStreamBlocksRows) return fail(UGBSA_EARG, "N=%d gives %d key blocks; the per-row selector holds at most %d", N, nb, ugbsa::kStreamBlocksRows);
  if (k_eff < 0 || k_eff >= nb) return fail(UGBSA_EARG, "k_eff=%d out of range [0, NB=%d)", k_eff, nb);
  if (k_eff > 0 && margin == nullptr) return fail(UGBSA_EARG, "margin is null (k_eff > 0)");
  int K;
  if (policy == UGBSA_V1_BELIEF) {
    if (k_min < 0 || k_max < 1 || !(top_p == top_p)) return fail(UGBSA_EARG, "belief needs k_max >= 1 and a top_p");
    K = k_max < nb ? k_max : nb;
  } else {
    if (k_bud < 1 || k_bud > nb) return fail(UGBSA_EARG, "k_bud=%d out of range [1, NB=%d]", k_bud, nb);
    K = k_bud;
  }
  if (k_eff + 1 > K) K = k_eff + 1;
  if (K > ugbsa::kMaxSlots) return fail(UGBSA_EARG, "ranking %d blocks deep exceeds %d", K, ugbsa::kMaxSlots);
  const int64_t per_row = static_cast<int64_t>(B) * H * nb;
  const int64_t chunk_tiles = workspace_elems / (per_row * ugbsa::kBlock);
  if (chunk_tiles < 1) {
    if (workspace == nullptr)
      return fail(UGBSA_EARG, "select_mask_static: one 64-row tile needs B*H*64*NB = %lld fp32, beyond the %lld of the static scratch",
                  (long long)(per_row * ugbsa::kBlock), (long long)workspace_elems);
    return fail(UGBSA_EARG, "workspace of %lld floats holds less than one 64-row tile (%lld)", (long long)workspace_elems, (long long)(per_row * ugbsa::kBlock));
  }
  if (workspace == nullptr) {   // the static scratch of this device (sizes checked above)
    rc = static_scratch(&workspace);
    if (rc) return rc;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Qt = (M + ugbsa::kBlock - 1) / ugbsa::kBlock;
  for (int t0 = 0; t0 < Qt; t0 += static_cast<int>(chunk_tiles)) {
    const int t1 = t0 + static_cast<int>(chunk_tiles) < Qt ? t0 + static_cast<int>(chunk_tiles) : Qt;
    ugbsa::SelectAux aux;
    aux.row_scores = workspace;
    aux.rows_t0 = t0;
    aux.rows_t1 = t1;
    hipError_t e = ugbsa::launch_select(static_cast<const uint16_t*>(q), sq_b, sq_h, sq_m,
                                        static_cast<const uint16_t*>(planes), B, H, Hk, M, N, D,
                                        dtype, mode, scaling, 1, 1, 0, nullptr, nullptr, nullptr, st, &aux);
    if (e != hipSuccess) return hip_result(e, "select_mask row scores");
    ugbsa::RowsArgs a;
    a.scores = workspace;
    a.r0 = t0 * ugbsa::kBlock;
    a.nrows = (t1 - t0) * ugbsa::kBlock;
    a.B = B; a.H = H; a.M = M; a.NB = nb;
    a.K = K;
    a.k_bud = k_bud;
    a.belief = policy == UGBSA_V1_BELIEF;
    a.top_p = top_p;
    a.k_min = k_min; a.k_max = k_max;
    a.k_eff = k_eff;
    a.penalty = penalty;
    a.keep = keep;
    a.margin = k_eff > 0 ? margin : nullptr;
    e = ugbsa::launch_select_rows(a, st);
    if (e != hipSuccess) return hip_result(e, "select_mask rows");
  }
  return hip_result(hipSuccess, "select_mask");
}

int attn_fwd_common(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                    const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                    const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                    const int32_t* kv_idx, const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                    int64_t si_t, int64_t si_s, int B, int H, int Hk, int M, int N, int D,
                    int dtype, int Qt, int k_slots, int block_m, float scale, void* out,
                    int64_t so_b, int64_t so_h, int64_t so_m, int64_t so_d, void* workspace,
                    int64_t workspace_elems, void* stream) {
  int rc = check_dims(B, H, Hk, D, dtype);
  if (rc) return rc;
  if ((rc = check_bf16_operand("q", q, sq_b, sq_h, sq_m, sq_d))) return rc;
  if ((rc = check_bf16_operand("k", k, sk_b, sk_h, sk_n, sk_d))) return rc;
  if (v != nullptr && (rc = check_bf16_operand("v", v, sv_b, sv_h, sv_n, sv_d))) return rc;
  if (out == nullptr) return fail(UGBSA_EARG, "out is null");
  if (so_d != 1 || (reinterpret_cast<uintptr_t>(out) & 7u) || so_b % 4 || so_h % 4 || so_m % 4)
    return fail(UGBSA_ELAYOUT, "out: head_dim stride 1, 8-byte aligned rows required");
  if (kv_idx == nullptr || si_s != 1) return fail(UGBSA_ELAYOUT, "kv_idx must be non-null with unit slot stride");
  if (workspace == nullptr || !aligned16(workspace)) return fail(UGBSA_EARG, "workspace (K/V operand copies) must be a 16-byte aligned buffer");
  if (M < 1 || N < 1) return fail(UGBSA_EARG, "M and N must be positive");
  // K/V operand copies, then the tile schedule the launch writes
  if (workspace_elems < ugbsa_attn_workspace_elems(B, Hk, N, D))
    return fail(UGBSA_EARG, "workspace of %lld elements is smaller than ugbsa_attn_workspace_elems (%lld)",
                (long long)workspace_elems, (long long)ugbsa_attn_workspace_elems(B, Hk, N, D));
  // the causal mask takes query row i as key position i (one-shot prefill)
  if (M != N) return fail(UGBSA_EARG, "attention needs query length == key length (M=%d, N=%d)", M, N);
  if (block_m != 64 && block_m != 32) return fail(UGBSA_EARG, "block_m must be 64 or 32 (got %d)", block_m);
  if (Qt != (M + block_m - 1) / block_m) return fail(UGBSA_EARG, "kv_idx holds %d tiles, M=%d needs %d", Qt, M, (M + block_m - 1) / block_m);
  if (k_slots < 1) return fail(UGBSA_EARG, "k_slots must be positive");
  if (!(scale != 0.f && scale - scale == 0.f)) return fail(UGBSA_EARG, "scale must be finite and nonzero");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint16_t* vt = static_cast<uint16_t*>(workspace);
  if (static_cast<int64_t>(N) * sk_n * 2 > 0xFFFFFFFFLL || kv_copy_elems(1, 1, N, D) * 2 > 0xFFFFFFFFLL)
    return fail(UGBSA_EARG, "one KV head's K rows exceed the 4 GiB buffer-load range");
  if (k_slots > 16384 && block_m == 64 && D <= 128)
    return fail(UGBSA_EARG, "k_slots=%d exceeds the 16384-slot kv list of the attention kernel", k_slots);
  if (rowmask != nullptr && k_slots > 8192 && block_m == 64 && D <= 128)
    return fail(UGBSA_EARG, "k_slots=%d exceeds the 8192-slot kv list of the row-masked attention kernel", k_slots);
  if (v != nullptr) {   // NULL: the workspace already holds ugbsa_attn_prepare_kv's output
    hipError_t e = ugbsa::launch_attn_prepare(static_cast<const uint16_t*>(k), sk_b, sk_h, sk_n,
                                              static_cast<const uint16_t*>(v), sv_b, sv_h, sv_n,
                                              B, Hk, N, D, block_m, vt, st);
    if (e != hipSuccess) return hip_result(e, "attn_prepare_kv");
  }
  return hip_result(ugbsa::launch_attn_fwd(static_cast<const uint16_t*>(q), sq_b, sq_h, sq_m,
                                           static_cast<const uint16_t*>(k), sk_b, sk_h, sk_n, vt,
                                           kv_idx, si_b, si_h, si_t, B, H, Hk, M, N, D, dtype, Qt,
                                           k_slots, block_m, scale, static_cast<uint16_t*>(out),
                                           so_b, so_h, so_m, st, rowmask,
                                           reinterpret_cast<int32_t*>(vt + kv_copy_elems(B, Hk, N, D))),
                    "attn_fwd");
}

}  // namespace

extern "C" {

int ugbsa_attn_fwd(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                   const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                   const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                   const int32_t* kv_idx, int64_t si_b, int64_t si_h, int64_t si_t,
                   int64_t si_s, int B, int H, int Hk, int M, int N, int D, int dtype, int Qt,
                   int k_slots, int block_m, float scale, void* out, int64_t so_b,
                   int64_t so_h, int64_t so_m, int64_t so_d, void* workspace,
                   int64_t workspace_elems, void* stream) {
  return attn_fwd_common(q, sq_b, sq_h, sq_m, sq_d, k, sk_b, sk_h, sk_n, sk_d, v, sv_b, sv_h,
                         sv_n, sv_d, kv_idx, nullptr, si_b, si_h, si_t, si_s, B, H, Hk, M, N, D,
                         dtype, Qt, k_slots, block_m, scale, out, so_b, so_h, so_m, so_d,
                         workspace, workspace_elems, stream);
}

int ugbsa_attn_fwd_rows(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                        const void* k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sk_d,
                        const void* v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t sv_d,
                        const int32_t* kv_idx, const uint64_t* rowmask, int64_t si_b,
                        int64_t si_h, int64_t si_t, int64_t si_s, int B, int H, int Hk, int M,
                        int N, int D, int dtype, int Qt, int k_slots, int block_m, float scale,
                        void* out, int64_t so_b, int64_t so_h, int64_t so_m, int64_t so_d,
                        void* workspace, int64_t workspace_elems, void* stream) {
  if (rowmask == nullptr) return fail(UGBSA_EARG, "rowmask is null");
  return attn_fwd_common(q, sq_b, sq_h, sq_m, sq_d, k, sk_b, sk_h, sk_n, sk_d, v, sv_b, sv_h,
                         sv_n, sv_d, kv_idx, rowmask, si_b, si_h, si_t, si_s, B, H, Hk, M, N, D,
                         dtype, Qt, k_slots, block_m, scale, out, so_b, so_h, so_m, so_d,
                         workspace, workspace_elems, stream);
}

int ugbsa_keep_kv_idx(const uint8_t* keep, int B, int H, int M, int NB, int block_m,
                      int32_t* kv_idx, uint64_t* rowmask, int32_t* counts, void* stream) {
  if (keep == nullptr || kv_idx == nullptr || counts == nullptr)
    return fail(UGBSA_EARG, "keep / kv_idx / counts is null");
  if (B < 1 || H < 1 || M < 1 || NB < 1) return fail(UGBSA_EARG, "B, H, M, NB must be positive");
  if (block_m != 64 && block_m != 32) return fail(UGBSA_EARG, "block_m must be 64 or 32 (got %d)", block_m);
  return hip_result(ugbsa::launch_keep_kv_idx(keep, B, H, M, NB, block_m, kv_idx, rowmask, counts,
                                              static_cast<hipStream_t>(stream)),
                    "keep_kv_idx");
}

int64_t ugbsa_select_mask_workspace_elems(int B, int H, int M, int N) {
  const int64_t nb = (N + ugbsa::kBlock - 1) / ugbsa::kBlock;
  const int64_t mp = (M + ugbsa::kBlock - 1) / ugbsa::kBlock * ugbsa::kBlock;
  return static_cast<int64_t>(B) * H * mp * nb;
}

int ugbsa_select_mask(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m, int64_t sq_d,
                      const void* planes, int B, int H, int Hk, int M, int N, int D, int dtype,
                      int mode, float scaling, int policy, int k_bud, int k_eff, int k_min,
                      int k_max, float top_p, const float* penalty, float* workspace,
                      int64_t workspace_elems, uint8_t* keep, float* margin, void* stream) {
  if (workspace == nullptr) return fail(UGBSA_EARG, "workspace is null");
  return select_mask_impl(q, sq_b, sq_h, sq_m, sq_d, planes, B, H, Hk, M, N, D, dtype, mode,
                          scaling, policy, k_bud, k_eff, k_min, k_max, top_p, penalty, workspace,
                          workspace_elems, keep, margin, stream);
}

int ugbsa_select_mask_static(const void* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                             int64_t sq_d, const void* planes, int B, int H, int Hk, int M, int N,
                             int D, int dtype, int mode, float scaling, int policy, int k_bud,
                             int k_eff, int k_min, int k_max, float top_p, const float* penalty,
                             uint8_t* keep, float* margin, void* stream) {
  return select_mask_impl(q, sq_b, sq_h, sq_m, sq_d, planes, B, H, Hk, M, N, D, dtype, mode,
                          scaling, policy, k_bud, k_eff, k_min, k_max, top_p, penalty, nullptr,
                          kStaticScratchFloats, keep, margin, stream);
}

int ugbsa_router_rows(const float* margin, int B, int H, int M, int NB, int grain, int rmode,
                      float tau, int64_t k_quant, int k_eff, uint8_t* keep, float* margin_eff,
                      uint8_t* uncertain, float* threshold, void* stream) {
  if (margin == nullptr || keep == nullptr || margin_eff == nullptr || uncertain == nullptr ||
      threshold == nullptr)
    return fail(UGBSA_EARG, "margin / keep / margin_eff / uncertain / threshold is null");
  if (B < 1 || H < 1 || M < 1 || NB < 1) return fail(UGBSA_EARG, "B, H, M, NB must be positive");
  if (grain != UGBSA_GRAIN_CELL && grain != UGBSA_GRAIN_ROW) return fail(UGBSA_EARG, "unknown router grain %d", grain);
  if (rmode != UGBSA_ROUTER_ABS && rmode != UGBSA_ROUTER_QUANTILE) return fail(UGBSA_EARG, "unknown router mode %d", rmode);
  const int64_t n = (grain == UGBSA_GRAIN_ROW ? 1 : static_cast<int64_t>(H)) * B * M;
  if (rmode == UGBSA_ROUTER_QUANTILE && (k_quant < 0 || k_quant > n))
    return fail(UGBSA_EARG, "k_quant=%lld out of range [0, %lld]", (long long)k_quant, (long long)n);
  if (k_eff < 1 || k_eff >= NB) return fail(UGBSA_EARG, "k_eff=%d out of range [1, NB=%d)", k_eff, NB);
  const int64_t row0 = static_cast<int64_t>(ugbsa::kBlock) * k_eff;   // first eligible row (M == N)
  return hip_result(ugbsa::launch_router_rows(margin, B, H, M, NB, grain, rmode, tau, k_quant,
                                              row0 < M ? static_cast<int>(row0) : M, keep,
                                              margin_eff, uncertain, threshold,
                                              static_cast<hipStream_t>(stream)),
                    "router_rows");
}

}  // extern "C"
