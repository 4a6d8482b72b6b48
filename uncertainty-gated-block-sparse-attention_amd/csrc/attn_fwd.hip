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
//   attn_fwd_pipe_kernel  64-row tiles (attn_pipe.h; head_dim 64 / 128 here,
//                         256 in attn_fwd256.hip): 32-key half blocks, S of
//                         the next half block computed while the softmax of
//                         the current one runs, K / V^T read from an
//                         operand-order copy (kv_operand_kernel);
//   attn_fwd_kernel       32-row tiles: K read in place, V^T from a
//                         per-block transposed copy (v_block_transpose_kernel).
//
// Launch order: the (b, t) tiles are ranked by their visited slots over all
// query heads (tile_work_kernel + tile_order_kernel, heaviest first), and the
// G query heads of one (b, KV head, t) are placed on the same XCD (workgroup
// i runs on XCD i % 8), so their shared picks (sink, local, group needles)
// hit the same L2; long contexts launch the units in generations
// (attn_pipe.h, launch_attn_pipe).

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

// Work of each (b, t) tile of 64 query rows: the visited slots of its
// kv_idx rows summed over the H query heads (slot values in [0, NB) and at
// most t, the blocks the attention loop visits).  One workgroup per tile:
// its four wavefronts take every fourth head, each lane every 64th slot, with
// the loads of four slots in flight at once; the partial counts meet in LDS.
__global__ __launch_bounds__(256) void tile_work_kernel(const int32_t* __restrict__ kv_idx,
                                                        int64_t si_b, int64_t si_h, int64_t si_t,
                                                        int B, int H, int Qt, int k_slots, int NB,
                                                        int32_t* __restrict__ work) {
  __shared__ int part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int bt = blockIdx.x;
  const int b = bt / Qt, t = bt - b * Qt;
  int cnt = 0;
  for (int h = wave; h < H; h += 4) {
    const int32_t* row = kv_idx + b * si_b + h * si_h + t * si_t;
    for (int s0 = lane; s0 < k_slots; s0 += 256) {
      int v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = s0 + 64 * j < k_slots ? row[s0 + 64 * j] : -1;
#pragma unroll
      for (int j = 0; j < 4; ++j) cnt += (v[j] >= 0 && v[j] < NB && v[j] <= t) ? 1 : 0;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
  if (lane == 0) part[wave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) work[bt] = part[0] + part[1] + part[2] + part[3];
}

// The (b, t) tiles ordered by work, heaviest first: a stable counting sort
// of the tiles, taken in the order t descending then b, by 16 work classes
// (class = work * 16 / (max work + 1)).  One workgroup: each thread takes a
// contiguous run of tiles, counts its classes, and after a scan over
// (class, thread) writes its tiles to their places.  order[i] = b * Qt + t.
constexpr int kOrderThreads = 512, kOrderClasses = 16;
__global__ __launch_bounds__(kOrderThreads) void tile_order_kernel(
    const int32_t* __restrict__ work, int B, int Qt, int32_t* __restrict__ order) {
  __shared__ int32_t cnt[kOrderClasses][kOrderThreads];
  __shared__ int32_t part[kOrderThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = B * Qt;
  const int per = (n + kOrderThreads - 1) / kOrderThreads;
  const int i0 = tid * per < n ? tid * per : n;
  const int i1 = i0 + per < n ? i0 + per : n;
  auto tile_at = [&](int i) -> int { return (i % B) * Qt + (Qt - 1 - i / B); };
  // the largest work
  int mx = 0;
  for (int i = i0; i < i1; ++i) mx = max(mx, work[tile_at(i)]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) part[wave] = mx;
  __syncthreads();
  mx = 0;
#pragma unroll
  for (int w = 0; w < kOrderThreads / 64; ++w) mx = max(mx, part[w]);
  auto cls = [&](int w) -> int {   // 0 = heaviest
    return kOrderClasses - 1 - static_cast<int>(static_cast<int64_t>(w) * kOrderClasses / (mx + 1));
  };
#pragma unroll
  for (int c = 0; c < kOrderClasses; ++c) cnt[c][tid] = 0;
  for (int i = i0; i < i1; ++i) ++cnt[cls(work[tile_at(i)])][tid];
  __syncthreads();
  // exclusive scan of cnt in (class, thread) order: thread j sums the
  // kOrderClasses consecutive counters [j * C, (j + 1) * C) of the flat array
  int32_t* flat = &cnt[0][0];
  int32_t loc[kOrderClasses];
  int sum = 0;
#pragma unroll
  for (int c = 0; c < kOrderClasses; ++c) {
    loc[c] = flat[tid * kOrderClasses + c];
    sum += loc[c];
  }
  __syncthreads();   // part[] is reused below
  const int excl = static_cast<int>(wave_excl_scan(static_cast<uint32_t>(sum), lane));
  if (lane == 63) part[wave] = excl + sum;
  __syncthreads();
  int base = excl;
  for (int w = 0; w < wave; ++w) base += part[w];
#pragma unroll
  for (int c = 0; c < kOrderClasses; ++c) {
    flat[tid * kOrderClasses + c] = base;
    base += loc[c];
  }
  __syncthreads();
  for (int i = i0; i < i1; ++i) {
    const int bt = tile_at(i);
    order[cnt[cls(work[bt])][tid]++] = bt;
  }
}

hipError_t launch_attn_tile_order(const int32_t* kv_idx, int64_t si_b, int64_t si_h,
                                  int64_t si_t, int B, int H, int Qt, int k_slots, int NB,
                                  int32_t* ws, hipStream_t stream) {
  const int n = B * Qt;
  tile_work_kernel<<<n, 256, 0, stream>>>(kv_idx, si_b, si_h, si_t, B, H, Qt, k_slots, NB, ws);
  tile_order_kernel<<<1, kOrderThreads, 0, stream>>>(ws, B, Qt, ws + n);
  return hipGetLastError();
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

// The 32-row tile kernel: a workgroup of WPT waves owns one Q tile of
// 16 * NT * WPT = 32 rows, each wave 16 * NT of them, and every wave visits
// every listed block.  V^T of the current block is requested before its S^T
// product and K of the next visited block right after it.
template <typename E, int D, int NT, int WPT>
__global__ __launch_bounds__(64 * WPT) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    const uint16_t* __restrict__ vt, const int32_t* __restrict__ kv_idx,
    const uint64_t* __restrict__ rowmask, int64_t si_b, int64_t si_h, int64_t si_t, int B,
    int Hk, int M, int N, int NB, int Qt, int k_slots, float scale_signed,
    uint16_t* __restrict__ out, int64_t so_b, int64_t so_h, int64_t so_m, int units, int grp) {
  constexpr int BM = 16 * NT * WPT, KS = D / 32, DT = D / 16;

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
  const uint16_t* qb = q + b * sq_b + h * sq_h;
  // A negative scale is moved onto Q (bf16 negation is exact), so the
  // softmax below always scales by scale_log2 > 0.
  const uint32_t qsign = scale_signed < 0.f ? 0x80008000u : 0u;
  const float scale_log2 = fabsf(scale_signed);

  // ---- Q (B operand of S^T) in registers ---------------------------------
  bf16x8 qf[NT][KS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + 16 * nt + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[nt][ks] = row < M ? __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4)) ^ qsign)
                           : zero_bf16x8();
  }

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

  auto block_at = [&](int s) -> int { return __builtin_amdgcn_readfirstlane(idx[s]); };
  auto visits = [&](int blk) -> bool { return blk >= 0 && blk < NB && blk * kBlock <= q_last; };
  auto next_slot = [&](int s) -> int {
    while (s < k_slots && !visits(block_at(s))) ++s;
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

  int s = next_slot(0);
  bf16x8 kf[4][KS];
  if (s < k_slots) load_k(block_at(s), kf);

  while (s < k_slots) {
    const int blk = block_at(s);
    const int kbase = blk * kBlock;
    bf16x8 vf[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) vf[dt][s2] = load_v(blk, dt, s2);

    // ---- S^T = K . Q^T -------------------------------------------------
    f32x4 st[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) st[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) st[mt][nt] = E::mfma(kf[mt][ks], qf[nt][ks], st[mt][nt]);

    const int s_next = next_slot(s + 1);
    if (s_next < k_slots) load_k(block_at(s_next), kf);

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
        w[0] = E::pack2(st[2 * s2][nt][0], st[2 * s2][nt][1]);
        w[1] = E::pack2(st[2 * s2][nt][2], st[2 * s2][nt][3]);
        w[2] = E::pack2(st[2 * s2 + 1][nt][0], st[2 * s2 + 1][nt][1]);
        w[3] = E::pack2(st[2 * s2 + 1][nt][2], st[2 * s2 + 1][nt][3]);
        pb[nt] = __builtin_bit_cast(bf16x8, w);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16x8 vv = vf[dt][s2];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[dt][nt] = E::mfma(vv, pb[nt], o[dt][nt]);
      }
    }
    s = s_next;
  }

  // ---- row sums, normalise and store ------------------------------------
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) l[nt] = quad_rows_sum(l[nt]);

  uint16_t* ob = out + b * so_b + h * so_h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float inv = l[nt] > 0.f ? 1.0f / l[nt] : 1.0f;
    const int row = row0 + 16 * nt + r16;
    if (row < M) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint32_t w0 = E::pack2(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
        const uint32_t w1 = E::pack2(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
        *reinterpret_cast<uint2*>(ob + row * so_m + 16 * dt + 4 * g4) = make_uint2(w0, w1);
      }
    }
  }
}

template <typename E, int D, int NT, int WPT>
static hipError_t launch_attn_t(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
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
  attn_fwd_kernel<E, D, NT, WPT><<<dim3(static_cast<unsigned>(wgs)), 64 * WPT, 0, stream>>>(
      q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, Hk, M,
      N, NB, Qt, k_slots, scale * kLog2e, out, so_b, so_h, so_m, units, grp);
  return hipGetLastError();
}

template <typename E>
static hipError_t launch_attn_fwd_e(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                    const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                    const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                                    int64_t si_h, int64_t si_t, int B, int H, int Hk, int M,
                                    int N, int D, int Qt, int k_slots, int block_m, float scale,
                                    uint16_t* out, int64_t so_b, int64_t so_h, int64_t so_m,
                                    hipStream_t stream, const uint64_t* rowmask,
                                    int32_t* order_ws) {
  if (uses_pipe(D, block_m)) {   // the pipelined kernel (its K/V operand layout is prepared)
    if (k_slots > kPipeMaxSlots) return hipErrorInvalidValue;
    const int NBk = (N + kBlock - 1) / kBlock;
    const int32_t* tile_order = nullptr;
    if (order_ws != nullptr) {
      hipError_t e = launch_attn_tile_order(kv_idx, si_b, si_h, si_t, B, H, Qt, k_slots, NBk,
                                            order_ws, stream);
      if (e != hipSuccess) return e;
      tile_order = order_ws + static_cast<int64_t>(B) * Qt;
    }
    if (D == 256)
      return launch_attn_pipe256(E::code, q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b,
                                 si_h, si_t, B, H, Hk, M, N, Qt, k_slots, scale, out, so_b, so_h,
                                 so_m, stream, tile_order);
    if (D == 128)
      return launch_attn_pipe<E, 128, 4, false, false>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
                                          rowmask, si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots,
                                          scale, out, so_b, so_h, so_m, stream, tile_order);
    return launch_attn_pipe<E, 64, 4, false, false>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx,
                                       rowmask, si_b, si_h, si_t, B, H, Hk, M, N, Qt, k_slots,
                                       scale, out, so_b, so_h, so_m, stream, tile_order);
  }
  // 32-row tiles: the older kernel (K read in place, V^T per block)
  if (block_m != 32) return hipErrorInvalidValue;
#define UGBSA_ATTN32_ARGS                                                                     \
  q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, H, Hk, M, \
      N, Qt, k_slots, scale, out, so_b, so_h, so_m, stream
  switch (D) {
    case 64: return launch_attn_t<E, 64, 2, 1>(UGBSA_ATTN32_ARGS);
    case 128: return launch_attn_t<E, 128, 2, 1>(UGBSA_ATTN32_ARGS);
    case 256: return launch_attn_t<E, 256, 1, 2>(UGBSA_ATTN32_ARGS);
  }
#undef UGBSA_ATTN32_ARGS
  return hipErrorInvalidValue;
}

hipError_t launch_attn_fwd(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                           const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                           const uint16_t* vt, const int32_t* kv_idx, int64_t si_b,
                           int64_t si_h, int64_t si_t, int B, int H, int Hk, int M, int N,
                           int D, int elem, int Qt, int k_slots, int block_m, float scale,
                           uint16_t* out, int64_t so_b, int64_t so_h, int64_t so_m,
                           hipStream_t stream, const uint64_t* rowmask, int32_t* order_ws) {
  if (elem == ElemF16::code)
    return launch_attn_fwd_e<ElemF16>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, si_b,
                                      si_h, si_t, B, H, Hk, M, N, D, Qt, k_slots, block_m, scale,
                                      out, so_b, so_h, so_m, stream, rowmask, order_ws);
  return launch_attn_fwd_e<ElemBf16>(q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, si_b,
                                     si_h, si_t, B, H, Hk, M, N, D, Qt, k_slots, block_m, scale,
                                     out, so_b, so_h, so_m, stream, rowmask, order_ws);
}

}  // namespace ugbsa
