// keep mask -> per-tile kv_idx and row masks (the v1 path's compaction).
//
// Restates _compute_kv_idx (src/triton_block_attn.py:125-146): per (b, h,
// Q tile of block_m rows) the blocks that any row of the tile keeps, in
// ascending order, padded with the sentinel NB, and their count (the host
// takes the maximum, as the reference's MAX_KEPT).  Rows past M are the
// reference's F.pad rows and keep nothing.  Beside each listed block it
// writes the mask of the tile rows that keep it (bit r: row t * block_m + r)
// — the per-row keep test of the reference kernel (:87-103), read by the
// attention kernels once per block instead of once per row.
//
// One wavefront per tile.  When rows are a multiple of 8 bytes (NB % 8 == 0,
// mask 8-byte aligned)
// a lane owns 8 consecutive blocks of each 512-block span and reads them as
// one 8-byte word per row (a row's span is one coalesced 512-byte read), ORs
// the row bits into 8 masks, and a wavefront prefix sum over the lanes'
// counts places the kept blocks in ascending order.  Otherwise 64 blocks at
// a time, one block per lane, with a ballot compaction.
#include "common.h"
#include "launch.h"

namespace ugbsa {

__global__ __launch_bounds__(256) void keep_kv_idx_kernel(
    const uint8_t* __restrict__ keep, int B, int H, int M, int NB, int block_m, int Qt,
    int32_t* __restrict__ kv_idx, uint64_t* __restrict__ rowmask, int32_t* __restrict__ counts) {
  const int lane = threadIdx.x & 63;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (unit >= static_cast<int64_t>(B) * H * Qt) return;
  const int64_t bh = unit / Qt;
  const int t = static_cast<int>(unit % Qt);
  const int rows = min(block_m, M - t * block_m);
  const uint8_t* kb = keep + (bh * M + static_cast<int64_t>(t) * block_m) * NB;
  int32_t* out = kv_idx + unit * NB;
  uint64_t* rm = rowmask != nullptr ? rowmask + unit * NB : nullptr;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int cnt = 0;
  if ((NB & 7) == 0 && (reinterpret_cast<uintptr_t>(keep) & 7) == 0) {
    for (int base = 0; base < NB; base += 512) {
      const int b0 = base + 8 * lane;
      uint64_t mk[8] = {0ull, 0ull, 0ull, 0ull, 0ull, 0ull, 0ull, 0ull};
      if (b0 < NB) {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(kb + b0);
        const int64_t stride = NB / 8;
        for (int r0 = 0; r0 < rows; r0 += 8) {
          uint64_t w[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) w[j] = r0 + j < rows ? src[(r0 + j) * stride] : 0ull;
#pragma unroll
          for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i)
              mk[i] |= static_cast<uint64_t>(((w[j] >> (8 * i)) & 0xFFull) != 0) << (r0 + j);
        }
      }
      int mine = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) mine += mk[i] != 0ull;
      int pos = cnt + static_cast<int>(wave_excl_scan(static_cast<uint32_t>(mine), lane));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (mk[i] != 0ull) {
          out[pos] = b0 + i;
          if (rm != nullptr) rm[pos] = mk[i];
          ++pos;
        }
      }
      cnt = __shfl(pos, 63, 64);
    }
  } else {
  for (int base = 0; base < NB; base += 64) {
    const int blk = base + lane;
    uint64_t mask = 0;
    if (blk < NB)
      for (int r = 0; r < rows; ++r)
        mask |= static_cast<uint64_t>(kb[static_cast<int64_t>(r) * NB + blk] != 0) << r;
    const bool ok = mask != 0;
    const uint64_t bal = __ballot(ok);
    if (ok) {
      const int pos = cnt + __popcll(bal & lt_mask);
      out[pos] = blk;
      if (rm != nullptr) rm[pos] = mask;
    }
    cnt += __popcll(bal);
  }
  }
  for (int s = cnt + lane; s < NB; s += 64) {
    out[s] = NB;
    if (rm != nullptr) rm[s] = 0ull;
  }
  if (lane == 0) counts[unit] = cnt;
}

hipError_t launch_keep_kv_idx(const uint8_t* keep, int B, int H, int M, int NB, int block_m,
                              int32_t* kv_idx, uint64_t* rowmask, int32_t* counts,
                              hipStream_t stream) {
  const int Qt = (M + block_m - 1) / block_m;
  const int64_t waves = static_cast<int64_t>(B) * H * Qt;
  keep_kv_idx_kernel<<<dim3(static_cast<unsigned>((waves + 3) / 4)), 256, 0, stream>>>(
      keep, B, H, M, NB, block_m, Qt, kv_idx, rowmask, counts);
  return hipGetLastError();
}

}  // namespace ugbsa
