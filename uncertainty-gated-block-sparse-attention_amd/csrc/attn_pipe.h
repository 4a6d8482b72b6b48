// The software-pipelined attention kernel over per-tile kv_idx (64-row
// tiles, one wavefront per tile), shared by the head_dim 64 / 128 builds
// (attn_fwd.hip) and the head_dim 256 build (attn_fwd256.hip, O^T in AGPRs).
#pragma once

#include "common.h"
#include "launch.h"

namespace ugbsa {

// The visited blocks are processed as 32-key half blocks u = 0, 1, ...
// (online softmax is exact at any key granularity).  Without SB (head_dim
// 64 / 128) step u overlaps
//   phase 1  MFMA: S^T(u+1) = K(u+1) . Q^T     ||  VALU: second half of
//                                                   P(u) = exp2(S(u) - m)
//   phase 2  MFMA: O^T += V^T(u) . P^T(u)      ||  VALU: first half of P(u+1)
// (row sums and bf16 packing included), with the VALU work woven between the
// MFMAs by hand.  The exp2 offsets m are lazy (kLazyLog2): a half block's P
// is computed with the current m, and only when some lane's sum of its P
// values exceeds 2^kLazyLog2 (commit) are the row maxima formed, l and O
// rescaled and P recomputed — after the first blocks a rare event.  K and
// V^T operands are prefetched into registers two half blocks ahead (K(u+3)
// is requested during phase 2, one 1 KiB slab per two MFMA pairs, V^T(u+2)
// two fragments at a time as the last row set's P.V MFMAs free them); the
// two S, K and V register sets alternate between consecutive steps (the loop
// is unrolled by 2).  Half blocks keep the live set at about 470 registers:
// O^T 128, two S 64, P 16, Q 64 (in AGPRs, read there by the MFMAs), two K
// 64, two V^T 64.
// With SB (head_dim 256) K / V^T keep one set each: K(u+2) requested after
// phase 1 and V^T(u+1) after phase 2, each a phase ahead of use; phase 1
// forms the second half of P(u) beside the S(u+1) MFMAs, and phase 2 forms
// the lane maxima of S(u+1), tests them against the lazy threshold and then
// forms the first half of P(u+1) (the rescale follows phase 2 when an offset
// moved).  Head_dim 256 (QLDS) doubles O^T, K and V^T, so Q moves to LDS and
// O^T (256 registers for 64 rows) to the AGPR file (OA), where only the P.V
// MFMAs touch it.
// The tile's kv_idx row is compacted into LDS once (visited blocks only), so
// sentinel and invisible slots cost nothing in the loop.
// Per-wave LDS bytes of attn_fwd_pipe_kernel: Q fragments (QLDS), block
// list, bitmap words and (with row masks) one mask per listed slot.
__host__ __device__ inline int pipe_wave_lds(int D, int NT, bool qlds, int k_slots, int NB,
                                             bool rowmask) {
  const int words = (NB + 31) / 32;
  int bytes = rowmask ? ((k_slots + words + 1) & ~1) * 4 + k_slots * 8 : (k_slots + words) * 4;
  if (qlds) bytes += NT * (D / 32) * 64 * 16;
  return (bytes + 15) / 16 * 16;
}

// Contexts of more than kGenBlocks key blocks run the attention units in
// generations (launch_attn_pipe).
constexpr int kGenBlocks = 512;

template <typename E, int D, int NT, bool QLDS, bool SB, bool OA>
__global__ __launch_bounds__(64 * (4 / NT)) void attn_fwd_pipe_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
    const uint16_t* __restrict__ vt, const int32_t* __restrict__ kv_idx,
    const uint64_t* __restrict__ rowmask, int64_t si_b, int64_t si_h, int64_t si_t, int B,
    int Hk, int M, int N, int NB, int Qt, int k_slots, float scale_log2,
    uint16_t* __restrict__ out, int64_t so_b, int64_t so_h, int64_t so_m,
    const int32_t* __restrict__ tile_order, int unit0, int unit_end, int grp) {
  constexpr int KS = D / 32, DT = D / 16, BM = 64;
  // NT = 4: one wavefront per 64-row tile; NT = 2: two wavefronts, 32 rows
  // each, which run independently (each keeps its own copy of the list)
  static_assert(NT == 4 || NT == 2, "a wavefront takes 64 or 32 rows of a tile");
  // OA: O^T accumulates in AGPRs (a 64-row tile at head_dim 256 fills all
  // 256 of them), written only by the P.V MFMAs of the SB loop
  static_assert(!OA || SB, "AGPR accumulators are used by the single-set loop");
  const int wave = threadIdx.x >> 6;
  // dynamic LDS per wave: [Q fragments (QLDS)] [block list] [bitmap] [row masks]
  extern __shared__ __align__(16) unsigned char psm_all[];
  unsigned char* psm = psm_all + wave * pipe_wave_lds(D, NT, QLDS, k_slots, NB, rowmask != nullptr);
  constexpr int QBYTES = QLDS ? NT * KS * 64 * 16 : 0;
  int32_t* blist = reinterpret_cast<int32_t*>(psm + QBYTES);

  // Workgroup -> unit (one (b, t) tile of one KV head g) and query head of
  // the group.  Workgroup i runs on XCD i % 8: the grp heads of a unit share
  // an XCD, and a launch's units land on the XCDs round robin, so with Hk
  // dividing 8 every XCD serves one KV head.  Tiles come heaviest first:
  // from tile_order (a launch covers units [unit0, unit_end)), or by t
  // descending.  In the generations of head_dim 256 (below) each XCD takes
  // one contiguous run of the launch's tiles instead (XCD x: KV head x % Hk,
  // run x / Hk of n / 8 tiles): neighbouring tiles list mostly the same
  // blocks, and a run of them keeps the XCD's L2 on fewer distinct 64 KiB
  // blocks (c5 attention 26.0 -> 24.2 ms; runs of 2 / 4 / 8 tiles dealt
  // round robin gain 0 / 1 / 3 %; head_dim 128 at 64K / 128K neither gains
  // nor loses).  Units stay a bijection: unit0 is a multiple of 8, so of Hk.
  const int wg = blockIdx.x;
  const int xcd = wg & 7;
  const int rest = wg >> 3;
  const int jh = rest % grp;
  int unit = unit0 + (rest / grp) * 8 + xcd;
  if constexpr (D > 128) {
    const int n = unit_end - unit0;
    if (tile_order != nullptr && NB > kGenBlocks && n % 8 == 0 && 8 % Hk == 0)
      unit = unit0 + ((xcd / Hk) * (n / 8) + rest / grp) * Hk + xcd % Hk;
  }
  if (unit >= unit_end) return;
  const int tile = unit / Hk, g = unit % Hk;
  int t, b;
  if (tile_order != nullptr) {
    const int bt = tile_order[tile];
    b = bt / Qt;
    t = bt - b * Qt;
  } else {
    t = Qt - 1 - tile / B;
    b = tile % B;
  }
  const int h = g * grp + jh;
  const int lane = threadIdx.x & 63;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int rbase = wave * 16 * NT;                  // this wave's first row in the tile
  const int row0 = t * BM + rbase;
  const int q_last = t * BM + BM - 1;

  // ---- Q tile requested first: its latency overlaps the list compaction ----
  const uint16_t* qb = q + b * sq_b + h * sq_h;
  // A negative scale is moved onto Q (bf16 negation is exact), so the
  // scores the softmax sees are always scaled by sl2 > 0.
  const float sl2 = fabsf(scale_log2);
  const uint32_t qsign = scale_log2 < 0.f ? 0x80008000u : 0u;
  u32x4 qraw[QLDS ? 1 : NT][QLDS ? 1 : KS];
  if constexpr (!QLDS) {
    // rows past M read row M - 1 (in bounds, no branch) and are zeroed below
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = min(row0 + 16 * nt + r16, M - 1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qraw[nt][ks] = __builtin_bit_cast(u32x4, load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4));
    }
  }

  // K and V^T operands of this KV head, in load order (kv_operand_kernel):
  // half block (blk, half) = K slabs at ((2 blk + half) * 2 * KS) KiB and
  // V^T slabs at ((2 blk + half) * DT) KiB; lane L reads 16 bytes at 16 L.
  const int64_t head_elems = static_cast<int64_t>(NB) * kBlock * D;
  const int64_t part = static_cast<int64_t>(B) * Hk * head_elems;
  const uint16_t* kop_head = vt + (static_cast<int64_t>(b) * Hk + g) * head_elems;
  const uint16_t* vop_head = kop_head + part;
  typedef bf16x8 KSet[2][KS];
  typedef bf16x8 VSet[DT];
  auto uni = [](int x) -> int { return __builtin_amdgcn_readfirstlane(x); };
  // Global (not buffer) loads: a wavefront streams K/V through the vector
  // memory pipeline faster with them, and every visited block lies inside
  // the operand copy, so no range check is needed.
  // First K / V^T slab of half block (blk, half), a wave-uniform address
  // (with blk uniform), and slab s of it for this lane: a scalar base plus a
  // 32-bit lane offset, so the loads take the SGPR-base form and no 64-bit
  // address per lane stays live in VGPRs.
  auto k_ptr = [&](int blk, int half) -> gchar* {
    return (gchar*)(kop_head) + static_cast<int64_t>(2 * blk + half) * (2 * KS * 1024);
  };
  auto v_ptr = [&](int blk, int half) -> gchar* {
    return (gchar*)(vop_head) + static_cast<int64_t>(2 * blk + half) * (DT * 1024);
  };
  uint32_t lane_b = static_cast<uint32_t>(lane) * 16u;
  auto slab = [&](gchar* base, int s) -> bf16x8 { return load_slab(base, lane_b, s); };
  auto load_k = [&](int blk, int half, KSet& kf) {
    gchar* p = k_ptr(blk, half);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[mt][ks] = slab(p, mt * KS + ks);
  };
  auto load_v = [&](int blk, int half, VSet& vf) {
    gchar* p = v_ptr(blk, half);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vf[dt] = slab(p, dt);
  };
  // The first operands are requested before the list is known, for block 0:
  // the visited blocks are ascending and the selector forces the sink block
  // 0 into every tile's list, so these loads overlap the list compaction.
  // A list that starts elsewhere requests its first block again below.
  // (Not with Q staged in LDS: at head_dim 256 it measured 1 % slower.)
  KSet ka, kb;
  VSet va, vb;
  if constexpr (!QLDS) {
    load_k(0, 0, ka);
    if constexpr (!SB) load_k(0, 1, kb);
    load_v(0, 0, va);
  }

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
  // four slot groups of 64 per round, their loads issued together (one
  // memory round trip per 256 slots instead of one per 64)
  for (int base0 = 0; base0 < k_slots; base0 += 256) {
    int blks[4];
    uint64_t mks[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = base0 + 64 * j + lane;
      blks[j] = s < k_slots ? idx[s] : -1;
      mks[j] = rmk != nullptr && s < k_slots ? rmk[s] : 0ull;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = blks[j];
      const bool ok = blk >= 0 && blk < NB && blk * kBlock <= q_last;
      const uint64_t bal = __ballot(ok);
      if (ok) {
        blist[nv + __popcll(bal & lt_mask)] = blk;
        if (rmk != nullptr) mlist[nv + __popcll(bal & lt_mask)] = mks[j];
        const uint32_t bit = 1u << (blk & 31);
        dup |= (atomicOr(&bits[blk >> 5], bit) & bit) != 0u;
      }
      nv += __popcll(bal);
    }
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
  bf16x8 qf[QLDS ? 1 : NT][QLDS ? 1 : KS];
  // With QLDS the fragments are staged once in LDS in operand order —
  // fragment (nt, ks) is one KiB with lane L's 16 bytes at 16 L — and read
  // back one fragment per MFMA pair (ds_read_b128, conflict-free), which
  // keeps Q (4 KS VGPRs a row set) out of the register file.
  bf16x8* qs = reinterpret_cast<bf16x8*>(psm);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + 16 * nt + r16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (QLDS) {
        const bf16x8 x = row < M ? __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4,
                                       load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4)) ^ qsign)
                                 : zero_bf16x8();
        qs[(nt * KS + ks) * 64 + lane] = x;
      } else {
        // Q lives in AGPRs for the whole tile: the MFMAs read their B
        // operand from there, where a VGPR copy would be spilled to AGPRs
        // and copied back (v_accvgpr_read) for every use
        const uint32_t keep = row < M ? 0xFFFFFFFFu : 0u;
        u32x4 xa = qraw[nt][ks];
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[i] = (xa[i] ^ qsign) & keep;
        asm volatile("" : "+a"(xa));
        qf[nt][ks] = __builtin_bit_cast(bf16x8, xa);
      }
    }
  }
  if constexpr (QLDS) wave_lds_sync();
  auto qfrag = [&](int nt, int ks) -> bf16x8 {
    if constexpr (QLDS) return qs[(nt * KS + ks) * 64 + lane];
    else return qf[nt][ks];
  };

  const int nu = 2 * nv;
  typedef f32x4 SBuf[2][NT];
  // Half block u (clamped to the last one) -> its block id (LDS read; the
  // caller applies readfirstlane where it needs the id, so the read can be
  // issued early) and its half.
  auto clamp_u = [&](int u) -> int { return min(u, nu - 1); };
  auto blk_raw = [&](int u) -> int { return blist[clamp_u(u) >> 1]; };

  f32x4 o[DT][NT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      o[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (OA) asm volatile("" : "+a"(o[dt][nt]));
    }
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
    if (kbase + 31 <= row0 && kbase + 32 <= N) {
      // causally visible and in bounds: only rows without the keep bit
      // drop, each as a whole row set of S
      if (mk != ~0ull) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const bool off = ((mk >> (rbase + 16 * nt + r16)) & 1ull) == 0;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (off) st[mt][nt][i] = -INFINITY;
        }
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int row = row0 + 16 * nt + r16;
        const bool off = ((mk >> (rbase + 16 * nt + r16)) & 1ull) == 0;
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
  // Lazy offsets with SB, tested lane-locally: a row's offset m only moves
  // when some lane's max of its raw scores exceeds
  // thr = (m + kLazyLog2) / sl2; the cross-lane row max is only formed inside
  // the (rare) rescale.  Without SB the row sums are tested instead (commit)
  // and lane maxima are formed only when that test fires.
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
  // With OA, every VALU access to O^T waits for the P.V MFMAs to retire.
  auto drain_o = [&]() {
    if constexpr (OA) {
      agpr_drain();
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) asm volatile("" : "+a"(o[dt][nt]));
    }
  };
  // The offset move itself (m, thr, l), leaving the factors for O in alpha.
  auto move_offsets = [&](float (&alpha)[NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float m_new = fmaxf(m[nt], quad_rows_max(rm[nt]) * sl2);
      alpha[nt] = __builtin_amdgcn_exp2f(m[nt] - m_new);
      m[nt] = m_new;
      thr[nt] = (m_new + kLazyLog2) * inv_sl2;
      l[nt] *= alpha[nt];
    }
  };
  auto scale_o = [&](const float (&alpha)[NT]) {
    drain_o();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        o[dt][nt] *= alpha[nt];
        // back into its AGPRs at once: left to the allocator, all 256
        // products would stay in VGPRs until the next MFMA reads them
        if constexpr (OA) asm volatile("" : "+a"(o[dt][nt]));
      }
  };
  auto rescale = [&]() {
    float alpha[NT];
    move_offsets(alpha);
    scale_o(alpha);
  };
  // Softmax element e of S (nt = e / 8): P = exp2(S * sl2 - m), the row sum
  // and the bf16 packing of P into pb (complete once element 8 nt + 7 is).
  float p[NT][8], sum[NT];
  uint32_t w[NT][4];
  auto softmax_elem = [&](const SBuf& st, int e) {
    const int nt = e / 8, kk = e % 8, mt = kk / 4, i = kk % 4;
    p[nt][kk] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][nt][i], sl2, -m[nt]));
    // the row sum and the packing take each exponential one element later: a
    // transcendental result read by the very next instruction costs a wait
    // state (c2 / c3 / c5 attention 0.4-0.6 % faster than adding at once)
    if (kk == 1) sum[nt] = p[nt][0];
    if (kk >= 2) sum[nt] += p[nt][kk - 1];
    if (kk >= 2 && (kk & 1) == 0) w[nt][kk / 2 - 1] = E::pack2(p[nt][kk - 2], p[nt][kk - 1]);
    if (kk == 7) {
      sum[nt] += p[nt][7];
      w[nt][3] = E::pack2(p[nt][6], p[nt][7]);
      if constexpr (SB) l[nt] += sum[nt];
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
          st[mt][nt] = E::mfma(kf[mt][ks], qfrag(nt, ks), ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[mt][nt]);
  };

  // The two phases of a step are woven by hand (one wave per SIMD issues in
  // order, so VALU work has to sit between the MFMAs of the instruction
  // stream); sched_barrier keeps the compiler from regrouping them.
  // With SB:
  //   phase 1: S^T(u+1) (NM1 MFMAs) || softmax of S(u) (all 8 NT elements)
  //   phase 2: O^T += V^T P^T(u) (NM2 MFMAs) || the row-max test of S(u+1)
  // Without SB:
  //   phase 1: S^T(u+1) || softmax elements [4 NT, 8 NT) of S(u)
  //   phase 2: O^T += V^T P^T(u) || softmax elements [0, 4 NT) of S(u+1)
  // with the lazy test after phase 1, on the row sums (commit).
  constexpr int NM1 = 2 * NT * KS, P1 = NM1 / 2;
  constexpr int E1ST = 4 * NT;                      // first softmax element of phase 1
  constexpr int NE1 = 8 * NT - E1ST;                // softmax elements of phase 1
  constexpr int NM2 = DT * NT, P2 = NM2 / 2;
  constexpr int RU = 4 * NT;                        // row-max units, spread over the P2 pairs
  auto phase1 = [&](const SBuf& cur, SBuf& nxt, const KSet& kf) {
    if constexpr (QLDS) {
      // pair j = (ks, nt): both M-tiles of fragment (nt, ks); the fragment
      // of pair j + 2 is requested in pair j, two MFMA pairs ahead of use.
      // Pairs run over the row sets two at a time (ks inside), so S(u+1)
      // comes into being two row sets at a time while the softmax of S(u)
      // frees its row sets in order: with OA that keeps the two S sets
      // within 48 live registers instead of 64.  Four accumulators cycle,
      // so a dependent MFMA issues 64 cycles after its predecessor.
      constexpr int NTG = NT >= 2 ? 2 : NT;         // row sets per group
      auto pair_nt = [](int j) { return (j / (NTG * KS)) * NTG + j % NTG; };
      auto pair_ks = [](int j) { return (j % (NTG * KS)) / NTG; };
      bf16x8 qr[3];
      qr[0] = qfrag(pair_nt(0), pair_ks(0));
      qr[1] = qfrag(pair_nt(1), pair_ks(1));
      static_for<P1>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        constexpr int ks = pair_ks(j), nt = pair_nt(j);
        if constexpr (j + 2 < P1) qr[(j + 2) % 3] = qfrag(pair_nt(j + 2), pair_ks(j + 2));
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
          nxt[mt][nt] = E::mfma(kf[mt][ks], qr[j % 3],
                                     ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : nxt[mt][nt]);
#pragma unroll
        for (int e = E1ST + (j * NE1 + P1 - 1) / P1; e < E1ST + ((j + 1) * NE1 + P1 - 1) / P1; ++e)
          softmax_elem(cur, e);
        __builtin_amdgcn_sched_barrier(0);
      });
    } else {
#pragma unroll
      for (int j = 0; j < P1; ++j) {
#pragma unroll
        for (int jj = 2 * j; jj < 2 * j + 2; ++jj) {
          const int ks = jj / (2 * NT), mt = (jj / NT) & 1, nt = jj % NT;
          nxt[mt][nt] = E::mfma(kf[mt][ks], qf[nt][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : nxt[mt][nt]);
        }
#pragma unroll
        for (int e = E1ST + (j * NE1 + P1 - 1) / P1; e < E1ST + ((j + 1) * NE1 + P1 - 1) / P1; ++e)
          softmax_elem(cur, e);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // O^T += V^T . P^T for MFMA pair j of phase 2 (jj = 2 j, 2 j + 1).
  auto pv_pair = [&](const VSet& vf, int j) {
    const int dt0 = (2 * j) / NT, nt0 = (2 * j) % NT, dt1 = (2 * j + 1) / NT, nt1 = (2 * j + 1) % NT;
    if constexpr (OA) {
      mfma16x16x32_agpr2<E>(o[dt0][nt0], vf[dt0], pb[nt0], o[dt1][nt1], vf[dt1], pb[nt1]);
    } else {
      o[dt0][nt0] = E::mfma(vf[dt0], pb[nt0], o[dt0][nt0]);
      o[dt1][nt1] = E::mfma(vf[dt1], pb[nt1], o[dt1][nt1]);
    }
  };
  // Phase 2 with SB: O^T += V^T . P^T(u) row set by row set (pairs over the
  // head dims of one row set, then the next), woven with the lazy test of
  // S(u+1) over the first row set's pairs and, once it has passed, the
  // first half of the softmax of S(u+1): row set nt' of P(u+1) is formed
  // in pb[nt'] once the MFMAs have read row set nt' of P(u).  When some
  // lane's maxima grew past the lazy bound the offsets move before any of
  // P(u+1) is formed (m, thr and l at once; O, which the MFMAs of this
  // phase still accumulate at the old offsets, is scaled by alpha after
  // the phase).  Returns whether O needs that scaling.
  auto phase2 = [&](const SBuf& nx, const VSet& vf, float (&alpha)[NT]) -> bool {
    constexpr int PPN = DT / 2, EPN = 8 / PPN;
    static_assert(PPN * (NT / 2 + 1) <= P2 && RU % PPN == 0, "phase 2 layout");
    grow = false;
    bool moved = false;
    static_for<P2>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int nt = (2 * j) / DT, dt0 = (2 * j) % DT;
      if constexpr (OA) {
        mfma16x16x32_agpr2<E>(o[dt0][nt], vf[dt0], pb[nt], o[dt0 + 1][nt], vf[dt0 + 1], pb[nt]);
      } else {
        o[dt0][nt] = E::mfma(vf[dt0], pb[nt], o[dt0][nt]);
        o[dt0 + 1][nt] = E::mfma(vf[dt0 + 1], pb[nt], o[dt0 + 1][nt]);
      }
      if constexpr (j < PPN) {
#pragma unroll
        for (int r = j * (RU / PPN); r < (j + 1) * (RU / PPN); ++r) rowmax_unit(nx, r);
      }
      if constexpr (j == PPN - 1) {
        // rare: the common path falls through (c5 attention 0.35 % faster; the
        // same hints on the head_dim-128 branches move Q out of the AGPRs and
        // spill 672 bytes per lane, 14x slower)
        if (__builtin_expect(__ballot(grow) != 0, 0)) {
          move_offsets(alpha);
          moved = true;
        }
      }
      if constexpr (j >= PPN && j < PPN * (NT / 2 + 1)) {
#pragma unroll
        for (int e = (j - PPN) * EPN; e < (j - PPN + 1) * EPN; ++e) softmax_elem(nx, e);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    return moved;
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
    for (int j = 0; j < P2; ++j) pv_pair(vf, j);
  };
  // Phase 2 without SB: the P.V MFMAs row set by row set; once
  // row set nt' of P(u) has been read, row set nt' of P(u+1) is computed
  // (elements 8 nt' .. 8 nt' + 7 of S(u+1), over the next DT / 2 pairs).
  // on_pair(j) issues this step's share of the next K loads before pair j,
  // after_pair(j) the V^T fragments pair j has read for the last time.
  auto phase2s = [&](const SBuf& nx, VSet& vf, auto&& on_pair, auto&& after_pair) {
    constexpr int PPN = DT / 2, EPN = 8 / PPN;
    static_assert(PPN * (NT / 2 + 1) <= P2, "row sets of P(u+1) fit in phase 2");
#pragma unroll
    for (int j = 0; j < P2; ++j) {
      on_pair(j);
#pragma unroll
      for (int jj = 2 * j; jj < 2 * j + 2; ++jj) {
        const int nt = jj / DT, dt = jj % DT;
        o[dt][nt] = E::mfma(vf[dt], pb[nt], o[dt][nt]);
      }
      after_pair(j);
      if (j >= PPN && j < PPN * (NT / 2 + 1)) {
#pragma unroll
        for (int e = (j - PPN) * EPN; e < (j - PPN + 1) * EPN; ++e) softmax_elem(nx, e);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The lazy test without SB, after the softmax of half block st
  // is complete: a lane's sum of its eight P values above 2^kLazyLog2 means
  // the offset m of that row is stale (some P exceeded the lazy bound).
  // Then the offsets move to the half block's row maxima, l and O are
  // rescaled and the softmax is redone — rare, as each move raises m by more
  // than kLazyLog2 - 3.  Otherwise every P is at most 2^kLazyLog2.  The row
  // sums enter l only after the test.
  const float big_sum = __builtin_exp2f(kLazyLog2);
  auto commit = [&](const SBuf& st) {
    bool big = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) big |= sum[nt] > big_sum;
    if (__ballot(big) != 0) {
      rowmax(st);
      rescale();
      softmax(st);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) l[nt] += sum[nt];
  };

  SBuf sa, sb;
  if constexpr (SB) {
    // One K and one V^T set (at head_dim 256 two would take 256 registers).
    // Step u: S(u) in cur (its first half already softmaxed), K(u+1) in ka,
    // V(u) in va; K(u+2) is requested after phase 1 and V(u+1) after
    // phase 2 — a phase ahead of use (about 2000 cycles at head_dim 256).
    auto step1 = [&](SBuf& cur, SBuf& nxt, int u) {
      const int rk = blk_raw(u + 2), rm1 = blk_raw(u + 1);
      asm volatile("" : "+v"(lane_b));
      phase1(cur, nxt, ka);
      load_k(uni(rk), clamp_u(u + 2) & 1, ka);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        u32x4 pin = __builtin_bit_cast(u32x4, pb[nt]);
        asm volatile("" : "+v"(pin), "+v"(l[nt]));
        pb[nt] = __builtin_bit_cast(bf16x8, pin);
      }
      mask(nxt, uni(rm1), (u + 1) & 1, mbits(u + 1));
      float alpha[NT];
      const bool moved = phase2(nxt, va, alpha);
      load_v(uni(rm1), (u + 1) & 1, va);
      if (__builtin_expect(moved, 0)) scale_o(alpha);
    };
    if (nv > 0) {
      const int b0 = uni(blk_raw(0));
      if (QLDS || b0 != 0) {
        load_k(b0, 0, ka);
        load_v(b0, 0, va);
      }
      qk(sa, ka);
      load_k(uni(blk_raw(1)), clamp_u(1) & 1, ka);
      mask(sa, uni(blk_raw(0)), 0, mbits(0));
      if (rowmax(sa)) rescale();
#pragma unroll
      for (int e = 0; e < E1ST; ++e) softmax_elem(sa, e);
      int u = 0;
      for (; u + 2 <= nu - 2; u += 2) {
        step1(sa, sb, u);
        step1(sb, sa, u + 1);
      }
      step1(sa, sb, u);
#pragma unroll
      for (int e = E1ST; e < 8 * NT; ++e) softmax_elem(sb, e);
      pv(va);
    }
  }
  // Step u: S(u) in cur, K(u+1) in kc, V(u) in vc; K(u+2) / V(u+1) in flight.
  auto step = [&](SBuf& cur, SBuf& nxt, KSet& kc, VSet& vc, int u) {
    // block ids of K(u+3), the mask of S(u+1) and V(u+2), read from LDS
    // before phase 1 so that their latency hides behind it
    const int rk = blk_raw(u + 3), rm1 = blk_raw(u + 1), rv = blk_raw(u + 2);
    phase1(cur, nxt, kc);
    commit(cur);
    gchar* kp = k_ptr(uni(rk), clamp_u(u + 3) & 1);
    // P and the row sums are only read later; pin them so that their
    // computation is not sunk past the mask branch into phase 2
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      u32x4 pin = __builtin_bit_cast(u32x4, pb[nt]);
      asm volatile("" : "+v"(pin), "+v"(l[nt]));
      pb[nt] = __builtin_bit_cast(bf16x8, pin);
    }
    mask(nxt, uni(rm1), (u + 1) & 1, mbits(u + 1));
    // K(u+3) into kc (free once phase 1 has read K(u+1)): one slab every
    // second MFMA pair of phase 2 (the odd ones) rather than all eight at
    // once, so the four waves of a CU do not load in bursts (c2 / c3 / c4
    // attention 1.0-1.4 % faster than the burst after phase 1, same box;
    // odd pairs 0.3 % faster than even ones)
    static_assert(P2 >= 4 * KS, "every K slab is requested within phase 2");
    // V^T(u+2) into vc, two fragments after each pair of the last row set
    // has read them for the last time (pair LAST + i reads fragments 2 i and
    // 2 i + 1), the final two after the phase: c3 / c4 attention 0.3-0.9 %
    // faster than all eight after the phase, c2 unchanged (same box)
    gchar* vp = v_ptr(uni(rv), clamp_u(u + 2) & 1);
    constexpr int LAST = P2 - DT / 2;
    phase2s(nxt, vc, [&](int j) {
      if ((j & 1) == 1 && j / 2 < 2 * KS) kc[(j / 2) / KS][(j / 2) % KS] = slab(kp, j / 2);
    }, [&](int j) {
      if (j >= LAST && j < P2 - 1) {
        vc[2 * (j - LAST)] = slab(vp, 2 * (j - LAST));
        vc[2 * (j - LAST) + 1] = slab(vp, 2 * (j - LAST) + 1);
      }
    });
#pragma unroll
    for (int dt = DT - 2; dt < DT; ++dt) vc[dt] = slab(vp, dt);
  };

  if (!SB && nv > 0) {
    // the loads are issued in the loop's order (K(u+1), V(u), K(u+2),
    // V(u+1) outstanding at each step), so that the wait counts the compiler
    // derives for the loop hold for its first iteration as for the others
    const int b0 = uni(blk_raw(0));
    if (QLDS || b0 != 0) {
      load_k(b0, 0, ka);
      load_k(b0, 1, kb);
      load_v(b0, 0, va);
    }
    qk(sa, ka);
    load_k(uni(blk_raw(2)), clamp_u(2) & 1, ka);
    load_v(uni(blk_raw(1)), 1, vb);
    mask(sa, uni(blk_raw(0)), 0, mbits(0));
    if (rowmax(sa)) rescale();
#pragma unroll
    for (int e = 0; e < E1ST; ++e) softmax_elem(sa, e);
    // nu = 2 * nv is even: steady steps u = 0 .. nu - 2, then the last half block.
    int u = 0;
    for (; u + 2 <= nu - 2; u += 2) {
      step(sa, sb, kb, va, u);
      step(sb, sa, ka, vb, u + 1);
    }
    step(sa, sb, kb, va, u);
#pragma unroll
    for (int e = E1ST; e < 8 * NT; ++e) softmax_elem(sb, e);
    commit(sb);
    pv(vb);
  }

  // ---- normalise and store ------------------------------------------------
  drain_o();
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
        const uint32_t w0 = E::pack2(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
        const uint32_t w1 = E::pack2(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
        *reinterpret_cast<uint2*>(ob + row * so_m + 16 * dt + 4 * g4) = make_uint2(w0, w1);
      }
    }
  }
}

// Resident workgroups of an attention kernel on the current device (the
// number one launch keeps in flight at once).
template <typename Kern>
static int resident_workgroups(Kern kern, int threads, size_t lds) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern),
                                                   threads, lds) != hipSuccess)
    return 0;
  return cus * per_cu;
}

// Units per launch.  Past kGenBlocks key blocks the units run in
// generations, one launch each, of a whole number of resident waves of
// workgroups: the units of a generation start together and sweep their
// ascending block lists in step, so a block that several tiles of a KV head
// list (the group's heads and the tiles around it pick many of the same
// blocks) is fetched into the XCD's L2 once for all of them.  Measured on
// MI355X, attention launch ms, one launch / generations of 1x / 2x / 3x / 4x
// the resident workgroups: c3 (128K, head_dim 128) 21.8 / 17.8 / 17.6 / 17.6
// / 17.5, 64K 9.4 / 9.4 / 9.5 / 9.2-9.3 / 9.2, c5 (128K, head_dim 256) 37.7
// / 27.6 / 28.2 / 29.1 / 29.8; at 32K (512 blocks, where L2 already holds
// 89 % of the re-reads) one launch, 2.13 against 2.30 / 2.23 / 2.20 / 2.19.
// The fabric traffic of the c3 launch falls from 120 GB to about 20 GB.  A
// fractional multiple leaves a partial last wave in every launch (x1.5:
// 22.4 ms at c3).
template <int D>
constexpr int gen_waves() { return D > 128 ? 1 : 3; }

// tile_order (optional): the (b, t) tiles heaviest first (attn_tile_order);
// it enables the generations above.  Without it, one launch with tiles by t
// descending.
template <typename E, int D, int NT, bool QLDS, bool SB, bool OA = false>
static hipError_t launch_attn_pipe(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                   const uint16_t* k, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                                   const uint16_t* vt, const int32_t* kv_idx,
                                   const uint64_t* rowmask, int64_t si_b, int64_t si_h,
                                   int64_t si_t, int B, int H, int Hk, int M, int N, int Qt,
                                   int k_slots, float scale, uint16_t* out, int64_t so_b,
                                   int64_t so_h, int64_t so_m, hipStream_t stream,
                                   const int32_t* tile_order = nullptr) {
  const int NB = (N + kBlock - 1) / kBlock;
  const int grp = H / Hk;
  const int units = B * Hk * Qt;
  constexpr int WPT = 4 / NT;
  const size_t lds = static_cast<size_t>(WPT) *
                     pipe_wave_lds(D, NT, QLDS, k_slots, NB, rowmask != nullptr);
  if (lds > 160 * 1024) return hipErrorInvalidConfiguration;
  auto kern = attn_fwd_pipe_kernel<E, D, NT, QLDS, SB, OA>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  // units per launch: gen_waves<D>() resident waves of workgroups, rounded
  // down to a multiple of 8 units (one per XCD)
  int gen = units;
  if (tile_order != nullptr && NB > kGenBlocks) {
    const int slots = resident_workgroups(kern, 64 * WPT, lds);
    gen = slots / grp / 8 * 8 * gen_waves<D>();
    if (gen < 8) gen = units;
  }
  for (int u0 = 0; u0 < units; u0 += gen) {
    const int n = units - u0 < gen ? units - u0 : gen;
    const int64_t wgs = 8LL * grp * ((n + 7) / 8);
    kern<<<dim3(static_cast<unsigned>(wgs)), 64 * WPT, lds, stream>>>(
        q, sq_b, sq_h, sq_m, k, sk_b, sk_h, sk_n, vt, kv_idx, rowmask, si_b, si_h, si_t, B, Hk,
        M, N, NB, Qt, k_slots, scale * kLog2e, out, so_b, so_h, so_m, tile_order, u0, u0 + n,
        grp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}


}  // namespace ugbsa
