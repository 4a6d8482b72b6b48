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
// inside a block so that each lane's eight P^T values are eight consecutive
// keys, which makes the V^T operand eight consecutive keys of one column.
//
// Two kernels share this mapping:
//   attn_fwd_pipe_kernel  64-row tiles at head_dim 64 / 128 (the default):
//                         32-key half blocks, S of the next half block
//                         computed while the softmax of the current one runs,
//                         K / V^T read from an operand-order copy
//                         (kv_operand_kernel) two half blocks ahead;
//   attn_fwd_kernel       head_dim 256 and 32-row tiles: K read in place,
//                         V^T from a per-block transposed copy
//                         (v_block_transpose_kernel); launch shape selectable.
//
// Launch order: heaviest tiles first (t descending; a tile visits up to
// min(t + 1, k_slots) blocks), and the G query heads of one (b, KV head, t)
// are placed on the same XCD (workgroup i runs on XCD i % 8), so their
// shared picks (sink, local, group needles) hit the same L2.
#include <cstdio>
#include <cstdlib>

#include "common.h"
#include "launch.h"
#include "attn_pipe.h"

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

// K and V of one 64-key block in the pipelined kernel's operand order: for
// each 32-key half block, K as 2 (mt) x KS 1 KiB slabs and V^T as DT 1 KiB
// slabs, where lane L's 16 bytes sit at 16 * L of its slab.  K slab (mt, ks)
// lane (g4, r16) = K[key 8 * (r16 >> 2) + 4 * mt + (r16 & 3)][32 * ks + 8 * g4 ..];
// V^T slab dt lane (g4, r16) = V[keys 8 * g4 .. 8 * g4 + 7][16 * dt + r16].
// Every operand load of the attention loop is then one contiguous KiB.
template <int D>
__global__ __launch_bounds__(256) void kv_operand_kernel(
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_h, int64_t sv_n, int Hk, int N,
    int NB, uint16_t* __restrict__ kop, uint16_t* __restrict__ vop) {
  constexpr int KS = D / 32, DT = D / 16, CH = D / 8, ROW = D + 8;
  // head_dim 256: K and V pass through one LDS tile in turn (two would
  // exceed 64 KiB of static LDS)
  constexpr bool ONE = D > 128;
  __shared__ __align__(16) uint16_t kt[kBlock][ROW];
  __shared__ __align__(16) uint16_t vt2[ONE ? 1 : kBlock][ROW];
  uint16_t (*vt_)[ROW] = ONE ? kt : vt2;
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const uint16_t* ks_ = k + b * sk_b + h * sk_h;
  const uint16_t* vs_ = v + b * sv_b + h * sv_h;
  auto stage = [&](bool with_k, bool with_v) {
    for (int i = threadIdx.x; i < kBlock * CH; i += 256) {
      const int r = i / CH, c = i % CH;
      const int key = blk * kBlock + r;
      u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
      if (key < N) {
        if (with_k) kv = *reinterpret_cast<const u32x4*>(ks_ + key * sk_n + c * 8);
        if (with_v) vv = *reinterpret_cast<const u32x4*>(vs_ + key * sv_n + c * 8);
      }
      if (with_k) *reinterpret_cast<u32x4*>(&kt[r][c * 8]) = kv;
      if (with_v) *reinterpret_cast<u32x4*>(&vt_[r][c * 8]) = vv;
    }
    __syncthreads();
  };
  stage(true, !ONE);
  const int64_t base = ((static_cast<int64_t>(b) * Hk + h) * NB + blk) * kBlock * D;
  // K: 2 halves x 2 mt x KS slabs x 64 lanes
  for (int i = threadIdx.x; i < 2 * 2 * KS * 64; i += 256) {
    const int lane = i & 63, slab = i >> 6;
    const int ks = slab % KS, mt = (slab / KS) & 1, half = slab / (2 * KS);
    const int g4 = lane >> 4, r16 = lane & 15;
    const int key = 32 * half + 8 * (r16 >> 2) + 4 * mt + (r16 & 3);
    *reinterpret_cast<u32x4*>(kop + base + static_cast<int64_t>(i) * 8) =
        *reinterpret_cast<const u32x4*>(&kt[key][32 * ks + 8 * g4]);
  }
  if (ONE) {
    __syncthreads();
    stage(false, true);
  }
  // V^T: 2 halves x DT slabs x 64 lanes
  for (int i = threadIdx.x; i < 2 * DT * 64; i += 256) {
    const int lane = i & 63, slab = i >> 6;
    const int dt = slab % DT, half = slab / DT;
    const int g4 = lane >> 4, r16 = lane & 15;
    i16x8 w;
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = static_cast<short>(vt_[32 * half + 8 * g4 + j][16 * dt + r16]);
    *reinterpret_cast<i16x8*>(vop + base + static_cast<int64_t>(i) * 8) = w;
  }
}

// The pipelined kernel serves 64-row tiles (head_dim 64 / 128 here, 256 in
// attn_fwd256.hip); 32-row tiles use attn_fwd_kernel, which reads K directly
// and V^T per block.
static bool uses_pipe(int D, int block_m) {
  return block_m == 64 && (D == 64 || D == 128 || D == 256);
}
// Longest kv_idx row the pipelined kernel compacts into LDS.
constexpr int kPipeMaxSlots = 16384;

hipError_t launch_attn_prepare(const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                               const uint16_t* v, int64_t sv_b, int64_t sv_h, int64_t sv_n,
                               int B, int Hk, int N, int D, int block_m, uint16_t* ws,
                               hipStream_t stream) {
  const int NB = (N + kBlock - 1) / kBlock;
  const int64_t part = static_cast<int64_t>(B) * Hk * NB * kBlock * D;
  dim3 grid(NB, Hk, B);
  if (uses_pipe(D, block_m)) {
    if (D == 64)
      kv_operand_kernel<64><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, v, sv_b, sv_h, sv_n, Hk, N, NB, ws, ws + part);
    else if (D == 128)
      kv_operand_kernel<128><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, v, sv_b, sv_h, sv_n, Hk, N, NB, ws, ws + part);
    else
      kv_operand_kernel<256><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, v, sv_b, sv_h, sv_n, Hk, N, NB, ws, ws + part);
    return hipGetLastError();
  }
  uint16_t* vt = ws + part;
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

// Launch shape of the attention kernel:
//   NT     16-row N-tiles per wave (a wave computes 16 * NT query rows);
//   WPT    waves per workgroup; a workgroup owns one Q tile;
//   SPLIT  true: every wave owns all 16 * NT rows of the tile and visits the
//          slots s = wave (mod WPT); the partial (m, l, O) of the waves are
//          merged through LDS at the end.  false: the waves own disjoint row
//          slices (tile = 16 * NT * WPT rows) and all visit every slot;
//   QLDS   Q fragments are staged once per tile in LDS and re-read per block
//          (frees 16 * NT * D / 64 VGPRs) instead of being held in registers;
//   PF     register prefetch: V^T of the current block is requested before
//          its S^T product and K of the next visited block right after it.
template <int D, int NT, int WPT, bool SPLIT, bool QLDS, bool PF>
struct AttnShape {
  static constexpr int BM = SPLIT ? 16 * NT : 16 * NT * WPT;
  static constexpr int KS = D / 32;
  static constexpr int DT = D / 16;
  static constexpr int QROW = D + 8;                  // padded LDS row (bank-conflict free)
  static constexpr int Q_BYTES = QLDS ? BM * QROW * 2 : 0;
  static constexpr int PART = (DT * NT * 4 + 2 * NT) * 64;   // floats per merged wave
  static constexpr int MERGE_BYTES = SPLIT ? (WPT - 1) * PART * 4 : 0;
  static constexpr int LDS = Q_BYTES > MERGE_BYTES ? Q_BYTES : MERGE_BYTES;
};

template <int D, int NT, int WPT, bool SPLIT, bool QLDS, bool PF>
__global__ __launch_bounds__(64 * WPT) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    const uint16_t* __restrict__ vt, const int32_t* __restrict__ kv_idx,
    const uint64_t* __restrict__ rowmask, int64_t si_b, int64_t si_h, int64_t si_t, int B,
    int Hk, int M, int N, int NB, int Qt, int k_slots, float scale_signed,
    uint16_t* __restrict__ out, int64_t so_b, int64_t so_h, int64_t so_m, int units, int grp) {
  using S = AttnShape<D, NT, WPT, SPLIT, QLDS, PF>;
  constexpr int BM = S::BM, KS = S::KS, DT = S::DT;
  extern __shared__ __align__(16) unsigned char smem[];

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
  const int row0 = t * BM + (SPLIT ? 0 : wave * 16 * NT);
  const uint16_t* qb = q + b * sq_b + h * sq_h;
  // A negative scale is moved onto Q (bf16 negation is exact), so the
  // softmax below always scales by scale_log2 > 0.
  const uint32_t qsign = scale_signed < 0.f ? 0x80008000u : 0u;
  const float scale_log2 = fabsf(scale_signed);

  // ---- Q (B operand of S^T): registers or LDS ---------------------------
  bf16x8 qf[QLDS ? 1 : NT][QLDS ? 1 : KS];
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem);
  if constexpr (QLDS) {
    constexpr int CH = D / 8;
    for (int pi = threadIdx.x; pi < BM * CH; pi += 64 * WPT) {
      const int r = pi / CH, c = pi % CH;
      const int row = t * BM + r;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (row < M) val = *reinterpret_cast<const u32x4*>(qb + row * sq_m + c * 8) ^ qsign;
      *reinterpret_cast<u32x4*>(qs + r * S::QROW + c * 8) = val;
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = row0 + 16 * nt + r16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[nt][ks] = row < M ? __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4)) ^ qsign)
                             : zero_bf16x8();
    }
  }
  const int qlds_row0 = (row0 - t * BM) + r16;    // this lane's first row inside the tile

  f32x4 o[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[NT], l[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) { m[nt] = -1e30f; l[nt] = 0.f; }

  const int64_t idx_off = b * si_b + h * si_h + t * si_t;
  const int32_t* idx = kv_idx + idx_off;
  // per-row keep masks of the listed blocks (bit r: tile row r keeps it), or
  // none: every row of the tile attends to every listed block
  const uint64_t* rmk = rowmask != nullptr ? rowmask + idx_off : nullptr;
  // K rows of this KV head: byte offsets past N * sk_n read as zeros.
  const __amdgpu_buffer_rsrc_t krs =
      make_rsrc(k + b * sk_b + g * sk_h, static_cast<uint32_t>(static_cast<int64_t>(N) * sk_n * 2));
  const int64_t vt_part = static_cast<int64_t>(B) * Hk * NB * D * kBlock;   // V^T after the K slot
  const __amdgpu_buffer_rsrc_t vrs =
      make_rsrc(vt + vt_part + (static_cast<int64_t>(b) * Hk + g) * NB * D * kBlock,
                static_cast<uint32_t>(static_cast<int64_t>(NB) * D * kBlock * 2));
  uint32_t koff[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
    koff[mt] = static_cast<uint32_t>(key_of(mt, r16) * sk_n * 2 + g4 * 16);
  const uint32_t voff = static_cast<uint32_t>(r16 * kBlock * 2 + g4 * 16);
  const int q_last = t * BM + BM - 1;
  constexpr int step = SPLIT ? WPT : 1;

  auto block_at = [&](int s) -> int { return __builtin_amdgcn_readfirstlane(idx[s]); };
  auto visits = [&](int blk) -> bool { return blk >= 0 && blk < NB && blk * kBlock <= q_last; };
  auto next_slot = [&](int s) -> int {
    while (s < k_slots && !visits(block_at(s))) s += step;
    return s;
  };
  auto load_k = [&](int blk, bf16x8 (&kf)[4][KS]) {
    const uint32_t sbase = static_cast<uint32_t>(blk * kBlock * sk_n * 2);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[mt][ks] = buffer_load_bf16x8(krs, koff[mt] + 64 * ks, sbase);
  };
  auto load_v = [&](int blk, int dt, int s2) -> bf16x8 {
    return buffer_load_bf16x8(vrs, voff + (16 * dt) * kBlock * 2 + 64 * s2,
                              static_cast<uint32_t>(blk * D * kBlock * 2));
  };

  int s = next_slot(SPLIT ? wave : 0);
  bf16x8 kf[4][KS];
  if (PF && s < k_slots) load_k(block_at(s), kf);

  while (s < k_slots) {
    const int blk = block_at(s);
    const int kbase = blk * kBlock;
    bf16x8 vf[PF ? DT : 1][2];
    if constexpr (PF) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) vf[dt][s2] = load_v(blk, dt, s2);
    } else {
      load_k(blk, kf);
    }

    // ---- S^T = K . Q^T -------------------------------------------------
    f32x4 st[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) st[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 qv[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        qv[nt] = QLDS ? *reinterpret_cast<const bf16x8*>(qs + (qlds_row0 + 16 * nt) * S::QROW + 32 * ks + 8 * g4)
                      : qf[QLDS ? 0 : nt][QLDS ? 0 : ks];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) st[mt][nt] = mfma16x16x32(kf[mt][ks], qv[nt], st[mt][nt]);
    }

    const int s_next = next_slot(s + step);
    if (PF && s_next < k_slots) load_k(block_at(s_next), kf);

    // ---- causal / bounds / row-keep mask, online softmax (log2 domain) ---
    uint64_t mk = ~0ull;
    if (rmk != nullptr) {
      const uint64_t x = rmk[s];
      mk = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x >> 32))) << 32) |
           static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
    }
    const bool need_mask = (kbase + kBlock - 1 > row0) || (kbase + kBlock > N) || mk != ~0ull;
    float mx_s[NT];
    bool grow = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = row0 + 16 * nt + r16;
      if (need_mask) {
        const bool off = ((mk >> (row - t * BM)) & 1ull) == 0;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kbase + 32 * (mt >> 1) + 8 * g4 + 4 * (mt & 1) + i;
            if (off || key > row || key >= N) st[mt][nt][i] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[mt][nt][i]);
      mx = quad_rows_max(mx);
      mx_s[nt] = mx * scale_log2;
      grow |= mx_s[nt] > m[nt] + kLazyLog2;
    }
    if (__ballot(grow)) {      // move the offsets (lazy: rarely after the first blocks)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float m_new = fmaxf(m[nt], mx_s[nt]);
        const float alpha = __builtin_amdgcn_exp2f(m[nt] - m_new);
        m[nt] = m_new;
        l[nt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][nt] *= alpha;
      }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float sum = 0.f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][nt][i], scale_log2, -m[nt]));
          st[mt][nt][i] = p;
          sum += p;
        }
      l[nt] += sum;
    }

    // ---- O^T += V^T . P^T ----------------------------------------------
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      bf16x8 pb[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        u32x4 w;
        w[0] = cvt_pk_bf16(st[2 * s2][nt][0], st[2 * s2][nt][1]);
        w[1] = cvt_pk_bf16(st[2 * s2][nt][2], st[2 * s2][nt][3]);
        w[2] = cvt_pk_bf16(st[2 * s2 + 1][nt][0], st[2 * s2 + 1][nt][1]);
        w[3] = cvt_pk_bf16(st[2 * s2 + 1][nt][2], st[2 * s2 + 1][nt][3]);
        pb[nt] = __builtin_bit_cast(bf16x8, w);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 vv = PF ? vf[PF ? dt : 0][s2] : load_v(blk, dt, s2);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[dt][nt] = mfma16x16x32(vv, pb[nt], o[dt][nt]);
      }
    }
    s = s_next;
  }

  // ---- row sums, cross-wave merge (SPLIT), normalise and store ----------
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    l[nt] = quad_rows_sum(l[nt]);
  }
  if constexpr (SPLIT) {
    float* part = reinterpret_cast<float*>(smem);
    __syncthreads();                       // every wave is done with the Q tile in LDS
    if (wave > 0) {
      float* my = part + (wave - 1) * S::PART;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int i = 0; i < 4; ++i) my[((dt * NT + nt) * 4 + i) * 64 + lane] = o[dt][nt][i];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        my[(DT * NT * 4 + nt) * 64 + lane] = m[nt];
        my[(DT * NT * 4 + NT + nt) * 64 + lane] = l[nt];
      }
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 1; w < WPT; ++w) {
      const float* pw = part + (w - 1) * S::PART;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float mw = pw[(DT * NT * 4 + nt) * 64 + lane];
        const float lw = pw[(DT * NT * 4 + NT + nt) * 64 + lane];
        const float mn = fmaxf(m[nt], mw);
        const float a0 = __builtin_amdgcn_exp2f(m[nt] - mn);
        const float a1 = __builtin_amdgcn_exp2f(mw - mn);
        m[nt] = mn;
        l[nt] = l[nt] * a0 + lw * a1;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            o[dt][nt][i] = o[dt][nt][i] * a0 + pw[((dt * NT + nt) * 4 + i) * 64 + lane] * a1;
      }
    }
  }

  uint16_t* ob = out + b * so_b + h * so_h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float inv = l[nt] > 0.f ? 1.0f / l[nt] : 1.0f;
    const int row = row0 + 16 * nt + r16;
    if (row < M) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint32_t w0 = cvt_pk_bf16(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
        const uint32_t w1 = cvt_pk_bf16(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
        *reinterpret_cast<uint2*>(ob + row * so_m + 16 * dt + 4 * g4) = make_uint2(w0, w1);
      }
    }
  }
}

template <int D, int NT, int WPT, bool SPLIT, bool QLDS, bool PF>
static hipError_t launch_attn_t(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                const uint16_t* vt, const int32_t* kv_idx,
                                const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                                int64_t si_t, int B, int H, int Hk, int M, int N, int Qt,
                                int k_slots, float scale, uint16_t* out, int64_t so_b,
                                int64_t so_h, int64_t so_m, hipStream_t stream) {
  using S = AttnShape<D, NT, WPT, SPLIT, QLDS, PF>;
  const int NB = (N + kBlock - 1) / kBlock;
  const int grp = H / Hk;
  const int units = B * Hk * Qt;
  const int64_t wgs = 8LL * grp * ((units + 7) / 8);
  auto kern = attn_fwd_kernel<D, NT, WPT, SPLIT, QLDS, PF>;
  if (S::LDS > 64 * 1024)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS);
  kern<<<dim3(static_cast<unsigned>(wgs)), 64 * WPT, S::LDS, stream>>>(
      q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, Hk, M,
      N, NB, Qt, k_slots, scale * kLog2e, out, so_b, so_h, so_m, units, grp);
  return hipGetLastError();
}

// Attention launch shapes, per (head_dim, tile rows).  The first entry of each
// group is the default; UGBSA_ATTN_VARIANT="NT,WPT,SPLIT,QLDS,PF" picks
// another compiled entry (tuning sweeps).
struct AttnVariant {
  int D, block_m, NT, WPT, SPLIT, QLDS, PF;
};
#define UGBSA_ATTN_VARIANTS(X)   \
  X(128, 64, 4, 1, 0, 0, 1)     \
  X(128, 64, 4, 1, 0, 0, 0)     \
  X(128, 64, 4, 2, 1, 1, 1)     \
  X(128, 64, 4, 2, 1, 1, 0)     \
  X(128, 64, 2, 2, 0, 0, 1)     \
  X(128, 64, 2, 2, 0, 1, 1)     \
  X(128, 64, 4, 4, 1, 1, 0)     \
  X(64, 64, 4, 1, 0, 0, 1)      \
  X(64, 64, 4, 2, 1, 1, 1)      \
  X(256, 64, 2, 2, 0, 0, 1)     \
  X(256, 64, 2, 2, 0, 1, 1)     \
  X(256, 64, 2, 2, 0, 1, 0)     \
  X(64, 32, 2, 1, 0, 0, 1)      \
  X(128, 32, 2, 1, 0, 0, 1)     \
  X(256, 32, 1, 2, 0, 0, 1)

hipError_t launch_attn_fwd(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                           const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                           const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                           int64_t si_h, int64_t si_t, int B, int H, int Hk, int M, int N,
                           int D, int Qt, int k_slots, int block_m, float scale, uint16_t* out,
                           int64_t so_b, int64_t so_h, int64_t so_m, hipStream_t stream,
                           const uint64_t* rowmask) {
  int want[5] = {-1, -1, -1, -1, -1};
  if (const char* env = getenv("UGBSA_ATTN_VARIANT"))
    sscanf(env, "%d,%d,%d,%d,%d", &want[0], &want[1], &want[2], &want[3], &want[4]);
  if (uses_pipe(D, block_m)) {   // the pipelined kernel (its K/V operand layout is prepared)
    if (k_slots > kPipeMaxSlots) return hipErrorInvalidValue;
    if (D == 256)
      return launch_attn_pipe256(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b,
                                 si_h, si_t, B, H, Hk, M, N, Qt, k_slots, scale, out, so_b, so_h,
                                 so_m, stream);
    // the single-set prefetch above kPipeLongBlocks context blocks;
    // UGBSA_PIPE_LONG=0/1 forces either variant (tests)
    const char* lv = getenv("UGBSA_PIPE_LONG");
    const bool long_ctx = lv != nullptr ? lv[0] == '1' : (N + kBlock - 1) / kBlock > kPipeLongBlocks;
    if (D == 128 && long_ctx)
      return launch_attn_pipe128_long(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
                                      rowmask, si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots,
                                      scale, out, so_b, so_h, so_m, stream);
    if (D == 128)
      return launch_attn_pipe<128, 4, false, false>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
                                          rowmask, si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots,
                                          scale, out, so_b, so_h, so_m, stream);
    return launch_attn_pipe<64, 4, false, false>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
                                       rowmask, si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots,
                                       scale, out, so_b, so_h, so_m, stream);
  }
  bool first = true;
#define UGBSA_TRY(D_, BM_, NT_, WPT_, SP_, QL_, PF_)                                            \
  if (D == D_ && block_m == BM_) {                                                             \
    const bool match = want[0] < 0 ? first                                                     \
        : (want[0] == NT_ && want[1] == WPT_ && want[2] == SP_ && want[3] == QL_ && want[4] == PF_); \
    first = false;                                                                             \
    if (match)                                                                                 \
      return launch_attn_t<D_, NT_, WPT_, SP_ != 0, QL_ != 0, PF_ != 0>(                        \
          q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, H, \
          Hk, M, N, Qt, k_slots, scale, out, so_b, so_h, so_m, stream);                        \
  }
  {
    UGBSA_ATTN_VARIANTS(UGBSA_TRY)
  }
#undef UGBSA_TRY
  return hipErrorInvalidValue;
}

}  // namespace ugbsa
