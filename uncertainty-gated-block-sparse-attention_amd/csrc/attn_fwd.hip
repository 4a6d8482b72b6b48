// Kernel 3: block-sparse causal attention over per-tile kv_idx, bf16 MFMA,
// fp32 online softmax, GQA (query head h reads KV head h / (H / Hk)).
//
// Semantics of the reference kernel src/triton_block_attn.py:203-264: for
// each (b, h, Q-tile t) visit the kv_idx slots in order, skip blk >= NB (the
// sentinel) and blocks starting after the tile's last row
// (t * BLOCK_M + BLOCK_M - 1), mask keys n > row or n >= N, update
// m / l / acc with P rounded to bf16 for the P.V product, write acc / l
// (l = 0 -> 1).  Negative slots are skipped too (the reference would read
// out of bounds).
//
// Mapping to CDNA4.  A wavefront owns 16 * NT query rows of one tile and
// computes the transposed products
//     S^T[key, row] = K . Q^T      (A = K rows, B = Q^T columns)
//     O^T[d, row]  += V^T . P^T    (A = V^T rows, B = P^T columns)
// with v_mfma_f32_16x16x32_bf16.  In this form every lane keeps its query
// row (lane & 15 of each 16-row N-tile) through both products, so the row
// max / row sum / rescale of the online softmax are lane-local plus two
// cross-lane steps, and P never leaves registers.  Keys are relabelled
// inside the 64-key block (pi below) so that each lane's eight P^T values
// are eight consecutive keys; V is pre-transposed per block ([NB][D][64],
// v_block_transpose_kernel) so both K and V^T operands are single 16-byte
// loads straight from global memory into MFMA operand registers.  There is
// no reuse of a K/V block between the waves of one tile that LDS staging
// could exploit at 64 rows per wave, so LDS is not used.
//
// Launch order: heaviest tiles first (t descending; a tile visits up to
// min(t + 1, k_slots) blocks), and the G query heads of one (b, KV head, t)
// are placed on the same XCD (workgroup i runs on XCD i % 8), so their
// shared picks (sink, local, group needles) hit the same L2.
#include "common.h"
#include "launch.h"

namespace ugbsa {

template <int D>
__global__ __launch_bounds__(256) void v_block_transpose_kernel(
    const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int Hk,
    int N, int NB, uint16_t* __restrict__ vt) {
  __shared__ uint16_t tile[kBlock][D + 8];
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const uint16_t* src = v + b * sv_b + h * sv_h;
  constexpr int CH = D / 8;
  for (int i = threadIdx.x; i < kBlock * CH; i += 256) {
    const int r = i / CH, c = i % CH;
    const int key = blk * kBlock + r;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (key < N) val = *reinterpret_cast<const u32x4*>(src + key * sv_n + c * 8);
    *reinterpret_cast<u32x4*>(&tile[r][c * 8]) = val;
  }
  __syncthreads();
  uint16_t* dst = vt + ((static_cast<int64_t>(b) * Hk + h) * NB + blk) * D * kBlock;
  for (int i = threadIdx.x; i < D * 8; i += 256) {
    const int d = i / 8, kc = i % 8;
    i16x8 w;
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = static_cast<short>(tile[kc * 8 + j][d]);
    *reinterpret_cast<i16x8*>(dst + d * kBlock + kc * 8) = w;
  }
}

hipError_t launch_v_block_transpose(const uint16_t* v, int64_t sv_b, int64_t sv_h, int64_t sv_n,
                                    int B, int Hk, int N, int D, uint16_t* vt,
                                    hipStream_t stream) {
  const int NB = (N + kBlock - 1) / kBlock;
  dim3 grid(NB, Hk, B);
  switch (D) {
    case 64: v_block_transpose_kernel<64><<<grid, 256, 0, stream>>>(v, sv_b, sv_h, sv_n, Hk, N, NB, vt); break;
    case 128: v_block_transpose_kernel<128><<<grid, 256, 0, stream>>>(v, sv_b, sv_h, sv_n, Hk, N, NB, vt); break;
    case 256: v_block_transpose_kernel<256><<<grid, 256, 0, stream>>>(v, sv_b, sv_h, sv_n, Hk, N, NB, vt); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Key (within its 64-key block) held by MFMA row R of S^T M-tile mt.
__device__ __forceinline__ int key_of(int mt, int R) {
  return 32 * (mt >> 1) + 8 * (R >> 2) + 4 * (mt & 1) + (R & 3);
}

template <int D, int NT, int WPT>
__global__ __launch_bounds__(64 * WPT) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    const uint16_t* __restrict__ vt, const int32_t* __restrict__ kv_idx, int64_t si_b,
    int64_t si_h, int64_t si_t, int B, int Hk, int M, int N, int NB, int Qt, int k_slots,
    float scale_log2, uint16_t* __restrict__ out, int64_t so_b, int64_t so_h, int64_t so_m,
    int units, int grp) {
  constexpr int BM = 16 * NT * WPT;  // rows per tile
  constexpr int KS = D / 32;         // contraction steps of S^T
  constexpr int DT = D / 16;         // 16-row tiles of O^T

  // Workgroup -> (unit, head-in-group); a unit is one (t, b, KV head).
  const int wg = blockIdx.x;
  const int xcd = wg & 7;
  const int rest = wg >> 3;
  const int jh = rest % grp;
  const int unit = (rest / grp) * 8 + xcd;
  if (unit >= units) return;
  const int per_t = B * Hk;
  const int t = Qt - 1 - unit / per_t;
  const int b = (unit % per_t) / Hk;
  const int g = (unit % per_t) % Hk;
  const int h = g * grp + jh;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int row0 = t * BM + wave * 16 * NT;

  bf16x8 qf[NT][KS];
  const uint16_t* qb = q + b * sq_b + h * sq_h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + 16 * nt + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[nt][ks] = row < M ? load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4) : zero_bf16x8();
  }

  f32x4 o[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[NT], l[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) { m[nt] = -1e30f; l[nt] = 0.f; }

  const int32_t* idx = kv_idx + b * si_b + h * si_h + t * si_t;
  const uint16_t* kb = k + b * sk_b + g * sk_h;
  const uint16_t* vb = vt + (static_cast<int64_t>(b) * Hk + g) * NB * D * kBlock;
  const int q_last = t * BM + BM - 1;

  for (int s = 0; s < k_slots; ++s) {
    const int blk = __builtin_amdgcn_readfirstlane(idx[s]);
    if (blk < 0 || blk >= NB || blk * kBlock > q_last) continue;
    const int kbase = blk * kBlock;

    // ---- S^T = K . Q^T -------------------------------------------------
    f32x4 st[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) st[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int key = kbase + key_of(mt, r16);
        const bf16x8 kf = key < N ? load_bf16x8(kb + key * sk_n + 32 * ks + 8 * g4) : zero_bf16x8();
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) st[mt][nt] = mfma16x16x32(kf, qf[nt][ks], st[mt][nt]);
      }
    }

    // ---- scale, causal / bounds mask, online softmax --------------------
    const bool need_mask = (kbase + kBlock - 1 > row0) || (kbase + kBlock > N);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = row0 + 16 * nt + r16;
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = st[mt][nt][i] * scale_log2;
          if (need_mask) {
            const int key = kbase + 32 * (mt >> 1) + 8 * g4 + 4 * (mt & 1) + i;
            if (key > row || key >= N) x = -INFINITY;
          }
          st[mt][nt][i] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const float m_new = fmaxf(m[nt], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[nt] - m_new);
      m[nt] = m_new;
      float sum = 0.f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(st[mt][nt][i] - m_new);
          st[mt][nt][i] = p;
          sum += p;
        }
      l[nt] = l[nt] * alpha + sum;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt][nt] *= alpha;
    }

    // ---- O^T += V^T . P^T ----------------------------------------------
    const uint16_t* vblk = vb + static_cast<int64_t>(blk) * D * kBlock;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      bf16x8 pb[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[i] = st[2 * s2][nt][i];
          f[4 + i] = st[2 * s2 + 1][nt][i];
        }
        pb[nt] = pack_bf16x8(f);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 vf = load_bf16x8(vblk + (16 * dt + r16) * kBlock + 32 * s2 + 8 * g4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[dt][nt] = mfma16x16x32(vf, pb[nt], o[dt][nt]);
      }
    }
  }

  // ---- normalise and store --------------------------------------------
  uint16_t* ob = out + b * so_b + h * so_h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float lt = l[nt];
    lt += shfl_xor_f(lt, 16);
    lt += shfl_xor_f(lt, 32);
    const float inv = lt > 0.f ? 1.0f / lt : 1.0f;
    const int row = row0 + 16 * nt + r16;
    if (row < M) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint32_t w0 = f32_to_bf16(o[dt][nt][0] * inv) | (static_cast<uint32_t>(f32_to_bf16(o[dt][nt][1] * inv)) << 16);
        const uint32_t w1 = f32_to_bf16(o[dt][nt][2] * inv) | (static_cast<uint32_t>(f32_to_bf16(o[dt][nt][3] * inv)) << 16);
        *reinterpret_cast<uint2*>(ob + row * so_m + 16 * dt + 4 * g4) = make_uint2(w0, w1);
      }
    }
  }
}

template <int D, int NT, int WPT>
static hipError_t launch_attn_t(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                                int64_t si_h, int64_t si_t, int B, int H, int Hk, int M, int N,
                                int Qt, int k_slots, float scale, uint16_t* out, int64_t so_b,
                                int64_t so_h, int64_t so_m, hipStream_t stream) {
  const int NB = (N + kBlock - 1) / kBlock;
  const int grp = H / Hk;
  const int units = B * Hk * Qt;
  const int64_t wgs = 8LL * grp * ((units + 7) / 8);
  attn_fwd_kernel<D, NT, WPT><<<dim3(static_cast<unsigned>(wgs)), 64 * WPT, 0, stream>>>(
      q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, si_b, si_h, si_t, B, Hk, M, N, NB,
      Qt, k_slots, scale * kLog2e, out, so_b, so_h, so_m, units, grp);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                           const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                           const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                           int64_t si_h, int64_t si_t, int B, int H, int Hk, int M, int N,
                           int D, int Qt, int k_slots, int block_m, float scale, uint16_t* out,
                           int64_t so_b, int64_t so_h, int64_t so_m, hipStream_t stream) {
#define UGBSA_ATTN(D_, NT_, WPT_)                                                          \
  return launch_attn_t<D_, NT_, WPT_>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, \
                                      si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots, scale, \
                                      out, so_b, so_h, so_m, stream)
  if (block_m == 64) {
    if (D == 64) UGBSA_ATTN(64, 4, 1);
    if (D == 128) UGBSA_ATTN(128, 4, 1);
    if (D == 256) UGBSA_ATTN(256, 2, 2);
  } else if (block_m == 32) {
    if (D == 64) UGBSA_ATTN(64, 2, 1);
    if (D == 128) UGBSA_ATTN(128, 2, 1);
    if (D == 256) UGBSA_ATTN(256, 1, 2);
  }
#undef UGBSA_ATTN
  return hipErrorInvalidValue;
}

}  // namespace ugbsa
