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
  __shared__ __align__(16) uint16_t kt[kBlock][ROW];
  __shared__ __align__(16) uint16_t vt_[kBlock][ROW];
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const uint16_t* ks_ = k + b * sk_b + h * sk_h;
  const uint16_t* vs_ = v + b * sv_b + h * sv_h;
  for (int i = threadIdx.x; i < kBlock * CH; i += 256) {
    const int r = i / CH, c = i % CH;
    const int key = blk * kBlock + r;
    u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (key < N) {
      kv = *reinterpret_cast<const u32x4*>(ks_ + key * sk_n + c * 8);
      vv = *reinterpret_cast<const u32x4*>(vs_ + key * sv_n + c * 8);
    }
    *reinterpret_cast<u32x4*>(&kt[r][c * 8]) = kv;
    *reinterpret_cast<u32x4*>(&vt_[r][c * 8]) = vv;
  }
  __syncthreads();
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

// The pipelined kernel serves 64-row tiles at head_dim 64 / 128; other
// shapes use attn_fwd_kernel, which reads K directly and V^T per block.
static bool uses_pipe(int D, int block_m) {
  return block_m == 64 && (D == 64 || D == 128);
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
    else
      kv_operand_kernel<128><<<grid, 256, 0, stream>>>(k, sk_b, sk_h, sk_n, v, sv_b, sv_h, sv_n, Hk, N, NB, ws, ws + part);
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

// Software-pipelined variant for 64-row tiles, one wavefront per tile.
//
// The visited blocks are processed as 32-key half blocks u = 0, 1, ...
// (online softmax is exact at any key granularity).  Step u overlaps
//   phase 1  MFMA: S^T(u+1) = K(u+1) . Q^T     ||  VALU: P(u) = exp2(S(u) - m),
//                                                   row sums, bf16 packing
//   phase 2  MFMA: O^T += V^T(u) . P^T(u)      ||  VALU: lane max of S(u+1)
//                                                   and the lazy-offset test
// with the VALU work woven between the MFMAs by hand.  The exp2 offsets m
// are lazy (kLazyLog2) and tested lane-locally; the cross-lane row max and
// the rescale of l and O run only when an offset must move, which after the
// first blocks is rare.  K and V^T operands are prefetched into registers
// two half blocks ahead (K(u+3) is requested after phase 1, V^T(u+2) after
// phase 2); the two S, K and V register sets alternate between consecutive
// steps (the loop is unrolled by 2).  Half blocks keep the live set at about
// 430 registers: O^T 128, two S 64, P 16, Q 64, two K 64, two V^T 64.  The
// tile's kv_idx row is compacted into LDS once (visited blocks only), so
// sentinel and invisible slots cost nothing in the loop.
template <int D, bool QLDS>
__global__ __launch_bounds__(64) void attn_fwd_pipe_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    const uint16_t* __restrict__ vt, const int32_t* __restrict__ kv_idx,
    const uint64_t* __restrict__ rowmask, int64_t si_b, int64_t si_h, int64_t si_t, int B,
    int Hk, int M, int N, int NB, int Qt, int k_slots, float scale_log2,
    uint16_t* __restrict__ out, int64_t so_b, int64_t so_h, int64_t so_m, int units, int grp) {
  constexpr int NT = 4, KS = D / 32, DT = D / 16, BM = 64;
  extern __shared__ int32_t blist[];        // k_slots entries (dynamic LDS)

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
  const int lane = threadIdx.x;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int row0 = t * BM;
  const int q_last = row0 + BM - 1;

  // ---- visited blocks of this tile, compacted into LDS in ascending order ---
  // (the heads of a KV group and neighbouring tiles then sweep shared blocks
  // together, which keeps them in L2).  A block listed twice in a row keeps
  // the slot order, so it is visited twice as the reference loop does.
  const int64_t idx_off = b * si_b + h * si_h + t * si_t;
  const int32_t* idx = kv_idx + idx_off;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  uint32_t* bits = reinterpret_cast<uint32_t*>(blist + k_slots);
  const int n_words = (min(t, NB - 1) >> 5) + 1;     // visible blocks are <= t
  // per-row keep masks of the visited blocks (bit r: tile row r keeps the
  // block), listed beside blist; without them every row attends every block
  const uint64_t* rmk = rowmask != nullptr ? rowmask + idx_off : nullptr;
  uint64_t* mlist = reinterpret_cast<uint64_t*>(
      blist + ((k_slots + (NB + 31) / 32 + 1) & ~1));
  for (int w = lane; w < n_words; w += 64) bits[w] = 0u;
  wave_lds_sync();
  int nv = 0;
  bool dup = false;
  for (int base = 0; base < k_slots; base += 64) {
    const int s = base + lane;
    const int blk = s < k_slots ? idx[s] : -1;
    const bool ok = blk >= 0 && blk < NB && blk * kBlock <= q_last;
    const uint64_t bal = __ballot(ok);
    if (ok) {
      blist[nv + __popcll(bal & lt_mask)] = blk;
      if (rmk != nullptr) mlist[nv + __popcll(bal & lt_mask)] = rmk[s];
      const uint32_t bit = 1u << (blk & 31);
      dup |= (atomicOr(&bits[blk >> 5], bit) & bit) != 0u;
    }
    nv += __popcll(bal);
  }
  wave_lds_sync();
  // with row masks the slots are visited in their order (the masks are
  // listed per slot); otherwise a list without repeats is re-sorted
  if (rmk == nullptr && __ballot(dup) == 0) {
    int pos = 0;
    for (int w0 = 0; w0 < n_words; w0 += 64) {
      const int w = w0 + lane;
      uint32_t word = w < n_words ? bits[w] : 0u;
      const uint32_t cnt = __popc(word);
      int at = pos + static_cast<int>(wave_excl_scan(cnt, lane));
      while (word) {
        const int j = __ffs(word) - 1;
        blist[at++] = w * 32 + j;
        word &= word - 1u;
      }
      pos = __shfl(at, 63, 64);
    }
    wave_lds_sync();
  }

  // ---- Q tile: MFMA B operands held in registers ---------------------------
  const uint16_t* qb = q + b * sq_b + h * sq_h;
  bf16x8 qf[NT][KS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + 16 * nt + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[nt][ks] = row < M ? load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4) : zero_bf16x8();
  }
  // A negative scale is moved onto Q (bf16 negation is exact), so the
  // scores the softmax sees are always scaled by sl2 > 0.
  const float sl2 = fabsf(scale_log2);
  if (scale_log2 < 0.f) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[nt][ks] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, qf[nt][ks]) ^ 0x80008000u);
  }

  // K and V^T operands of this KV head, in load order (kv_operand_kernel):
  // half block (blk, half) = K slabs at ((2 blk + half) * 2 * KS) KiB and
  // V^T slabs at ((2 blk + half) * DT) KiB; lane L reads 16 bytes at 16 L.
  const int64_t head_elems = static_cast<int64_t>(NB) * kBlock * D;
  const int64_t part = static_cast<int64_t>(B) * Hk * head_elems;
  const uint16_t* kop_head = vt + (static_cast<int64_t>(b) * Hk + g) * head_elems;
  const uint16_t* vop_head = kop_head + part;
  const int nu = 2 * nv;

  typedef bf16x8 KSet[2][KS];
  typedef bf16x8 VSet[DT];
  typedef f32x4 SBuf[2][NT];
  // Half block u (clamped to the last one) -> its block id (LDS read; the
  // caller applies readfirstlane where it needs the id, so the read can be
  // issued early) and its half.
  auto clamp_u = [&](int u) -> int { return min(u, nu - 1); };
  auto blk_raw = [&](int u) -> int { return blist[clamp_u(u) >> 1]; };
  auto uni = [](int x) -> int { return __builtin_amdgcn_readfirstlane(x); };
  // Global (not buffer) loads: a wavefront streams K/V through the vector
  // memory pipeline faster with them, and every visited block lies inside
  // the operand copy, so no range check is needed.
  auto load_k = [&](int blk, int half, KSet& kf) {
    const uint16_t* p = kop_head + static_cast<int64_t>(2 * blk + half) * (2 * KS * 512) + lane * 8;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[mt][ks] = load_bf16x8(p + (mt * KS + ks) * 512);
  };
  auto load_v = [&](int blk, int half, VSet& vf) {
    const uint16_t* p = vop_head + static_cast<int64_t>(2 * blk + half) * (DT * 512) + lane * 8;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vf[dt] = load_bf16x8(p + dt * 512);
  };

  f32x4 o[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[NT], l[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) { m[nt] = -1e30f; l[nt] = 0.f; }
  bf16x8 pb[NT];

  // Row-keep mask of half block u (wave-uniform), all rows without masks.
  auto mbits = [&](int u) -> uint64_t {
    if (rmk == nullptr) return ~0ull;
    const uint64_t x = mlist[clamp_u(u) >> 1];
    return (static_cast<uint64_t>(uni(static_cast<int>(x >> 32))) << 32) |
           static_cast<uint32_t>(uni(static_cast<int>(x)));
  };
  // Causal / bounds / row-keep mask (only half blocks crossing the diagonal
  // or N, or not kept by every row).
  auto mask = [&](SBuf& st, int blk, int half, uint64_t mk) {
    const int kbase = blk * kBlock + 32 * half;
    if ((kbase + 31 > row0) || (kbase + 32 > N) || mk != ~0ull) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int row = row0 + 16 * nt + r16;
        const bool off = ((mk >> (16 * nt + r16)) & 1ull) == 0;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kbase + 8 * g4 + 4 * mt + i;
            if (off || key > row || key >= N) st[mt][nt][i] = -INFINITY;
          }
      }
    }
  };
  // Lazy offsets, tested lane-locally: a row's offset m only moves when some
  // lane's max of its raw scores exceeds thr = (m + kLazyLog2) / sl2; the
  // cross-lane row max is only formed inside the (rare) rescale.
  float thr[NT], rm[NT], tm[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) thr[nt] = -INFINITY;
  const float inv_sl2 = 1.0f / sl2;
  // +inf in a register the optimiser cannot see through: med3(a, b, +inf) is
  // max(a, b) without the canonicalising copies that fmaxf of MFMA results
  // gets in IEEE mode.
  float pinf = INFINITY;
  asm volatile("" : "+v"(pinf));
  auto mx2 = [&](float a, float b) -> float { return __builtin_amdgcn_fmed3f(a, b, pinf); };
  bool grow = false;
  // Row-max unit r of S (nt = r / 4): stages 0-2 the max tree of the lane's
  // eight values, stage 3 the test against thr.
  auto rowmax_unit = [&](const SBuf& st, int r) {
    const int nt = r / 4, stage = r % 4;
    if (stage == 0) {
      tm[nt][0] = mx2(st[0][nt][0], st[0][nt][1]);
      tm[nt][1] = mx2(st[0][nt][2], st[0][nt][3]);
    } else if (stage == 1) {
      tm[nt][2] = mx2(st[1][nt][0], st[1][nt][1]);
      tm[nt][3] = mx2(st[1][nt][2], st[1][nt][3]);
    } else if (stage == 2) {
      tm[nt][0] = mx2(tm[nt][0], tm[nt][1]);
      tm[nt][2] = mx2(tm[nt][2], tm[nt][3]);
    } else {
      rm[nt] = mx2(tm[nt][0], tm[nt][2]);
      grow |= rm[nt] > thr[nt];
    }
  };
  // Move the offsets to the new row maxima (lane maxima rm -> row maxima)
  // and rescale l and O.
  auto rescale = [&]() {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float m_new = fmaxf(m[nt], quad_rows_max(rm[nt]) * sl2);
      const float alpha = __builtin_amdgcn_exp2f(m[nt] - m_new);
      m[nt] = m_new;
      thr[nt] = (m_new + kLazyLog2) * inv_sl2;
      l[nt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt][nt] *= alpha;
    }
  };
  // Softmax element e of S (nt = e / 8): P = exp2(S * sl2 - m), the row sum
  // and the bf16 packing of P into pb.
  float p[NT][8], sum[NT];
  uint32_t w[NT][4];
  auto softmax_elem = [&](const SBuf& st, int e) {
    const int nt = e / 8, kk = e % 8, mt = kk / 4, i = kk % 4;
    p[nt][kk] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][nt][i], sl2, -m[nt]));
    sum[nt] = kk == 0 ? p[nt][0] : sum[nt] + p[nt][kk];
    if (kk & 1) w[nt][kk / 2] = cvt_pk_bf16(p[nt][kk - 1], p[nt][kk]);
    if (kk == 7) {
      l[nt] += sum[nt];
      pb[nt] = __builtin_bit_cast(bf16x8, u32x4{w[nt][0], w[nt][1], w[nt][2], w[nt][3]});
    }
  };
  // S^T of one half block without interleaved work (prologue).
  auto qk = [&](SBuf& st, const KSet& kf) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          st[mt][nt] = mfma16x16x32(kf[mt][ks], qf[nt][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[mt][nt]);
  };

  // The two phases of a step are woven by hand (one wave per SIMD issues in
  // order, so VALU work has to sit between the MFMAs of the instruction
  // stream); sched_barrier keeps the compiler from regrouping them.
  //   phase 1: S^T(u+1) (NM1 MFMAs) || softmax of S(u) (32 elements a lane)
  //   phase 2: O^T += V^T P^T(u) (NM2 MFMAs) || the row-max test of S(u+1)
  constexpr int NM1 = 2 * NT * KS, P1 = NM1 / 2;
  constexpr int EPP = 8 * NT / P1;                  // softmax elements per MFMA pair
  constexpr int NM2 = DT * NT, P2 = NM2 / 2;
  constexpr int RPP = 4 * NT / P2;                  // row-max units per MFMA pair
  static_assert(EPP * P1 == 8 * NT && RPP * P2 == 4 * NT, "phase work must split evenly");
  auto phase1 = [&](const SBuf& cur, SBuf& nxt, const KSet& kf) {
#pragma unroll
    for (int j = 0; j < P1; ++j) {
#pragma unroll
      for (int jj = 2 * j; jj < 2 * j + 2; ++jj) {
        const int ks = jj / (2 * NT), mt = (jj / NT) & 1, nt = jj % NT;
        nxt[mt][nt] = mfma16x16x32(kf[mt][ks], qf[nt][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : nxt[mt][nt]);
      }
#pragma unroll
      for (int e = j * EPP; e < (j + 1) * EPP; ++e) softmax_elem(cur, e);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto phase2 = [&](const SBuf& nx, const VSet& vf) -> bool {
    grow = false;
#pragma unroll
    for (int j = 0; j < P2; ++j) {
#pragma unroll
      for (int jj = 2 * j; jj < 2 * j + 2; ++jj) {
        const int dt = jj / NT, nt = jj % NT;
        o[dt][nt] = mfma16x16x32(vf[dt], pb[nt], o[dt][nt]);
      }
#pragma unroll
      for (int r = j * RPP; r < (j + 1) * RPP; ++r) rowmax_unit(nx, r);
      __builtin_amdgcn_sched_barrier(0);
    }
    return __ballot(grow) != 0;
  };
  auto rowmax = [&](const SBuf& st) -> bool {
    grow = false;
#pragma unroll
    for (int r = 0; r < 4 * NT; ++r) rowmax_unit(st, r);
    return __ballot(grow) != 0;
  };
  // Softmax and P.V of the last half block (epilogue, not woven).
  auto softmax = [&](const SBuf& st) {
#pragma unroll
    for (int e = 0; e < 8 * NT; ++e) softmax_elem(st, e);
  };
  auto pv = [&](const VSet& vf) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[dt][nt] = mfma16x16x32(vf[dt], pb[nt], o[dt][nt]);
  };

  SBuf sa, sb;
  KSet ka, kb;
  VSet va, vb;
  // Step u: S(u) in cur, K(u+1) in kc, V(u) in vc; K(u+2) / V(u+1) in flight.
  auto step = [&](SBuf& cur, SBuf& nxt, KSet& kc, VSet& vc, int u) {
    // block ids of K(u+3), the mask of S(u+1) and V(u+2), read from LDS
    // before phase 1 so that their latency hides behind it
    const int rk = blk_raw(u + 3), rm1 = blk_raw(u + 1), rv = blk_raw(u + 2);
    phase1(cur, nxt, kc);
    load_k(uni(rk), clamp_u(u + 3) & 1, kc);
    // P and the row sums are only read later; pin them so that their
    // computation is not sunk past the mask branch into phase 2
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      u32x4 pin = __builtin_bit_cast(u32x4, pb[nt]);
      asm volatile("" : "+v"(pin), "+v"(l[nt]));
      pb[nt] = __builtin_bit_cast(bf16x8, pin);
    }
    mask(nxt, uni(rm1), (u + 1) & 1, mbits(u + 1));
    const bool moved = phase2(nxt, vc);
    load_v(uni(rv), clamp_u(u + 2) & 1, vc);
    if (moved) rescale();
  };

  if (nv > 0) {
    load_k(uni(blk_raw(0)), 0, ka);
    load_k(uni(blk_raw(1)), 1, kb);
    load_v(uni(blk_raw(0)), 0, va);
    load_v(uni(blk_raw(1)), 1, vb);
    qk(sa, ka);
    load_k(uni(blk_raw(2)), clamp_u(2) & 1, ka);
    mask(sa, uni(blk_raw(0)), 0, mbits(0));
    if (rowmax(sa)) rescale();
    // nu = 2 * nv is even: steady steps u = 0 .. nu - 2, then the last half block.
    int u = 0;
    for (; u + 2 <= nu - 2; u += 2) {
      step(sa, sb, kb, va, u);
      step(sb, sa, ka, vb, u + 1);
    }
    step(sa, sb, kb, va, u);
    softmax(sb);
    pv(vb);
  }

  // ---- normalise and store ------------------------------------------------
  uint16_t* ob = out + b * so_b + h * so_h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float lt = l[nt];
    lt = quad_rows_sum(lt);
    const float inv = lt > 0.f ? 1.0f / lt : 1.0f;
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

template <int D, bool QLDS>
static hipError_t launch_attn_pipe(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                   const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                   const uint16_t* vt, const int32_t* kv_idx,
                                   const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                                   int64_t si_t, int B, int H, int Hk, int M, int N, int Qt,
                                   int k_slots, float scale, uint16_t* out, int64_t so_b,
                                   int64_t so_h, int64_t so_m, hipStream_t stream) {
  const int NB = (N + kBlock - 1) / kBlock;
  const int grp = H / Hk;
  const int units = B * Hk * Qt;
  const int64_t wgs = 8LL * grp * ((units + 7) / 8);
  // block list, bitmap words, and (with row masks) one mask per listed slot
  size_t lds = static_cast<size_t>(k_slots) * 4 + static_cast<size_t>((NB + 31) / 32) * 4;
  if (rowmask != nullptr)
    lds = static_cast<size_t>((k_slots + (NB + 31) / 32 + 1) & ~1) * 4 + static_cast<size_t>(k_slots) * 8;
  auto kern = attn_fwd_pipe_kernel<D, QLDS>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  kern<<<dim3(static_cast<unsigned>(wgs)), 64, lds, stream>>>(
      q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, Hk, M,
      N, NB, Qt, k_slots, scale * kLog2e, out, so_b, so_h, so_m, units, grp);
  return hipGetLastError();
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
    if (D == 128)
      return launch_attn_pipe<128, false>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
                                          rowmask, si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots,
                                          scale, out, so_b, so_h, so_m, stream);
    return launch_attn_pipe<64, false>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
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
