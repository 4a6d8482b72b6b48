// Kernel 2: fused block scoring + tile max-pool + top-k + sigma margin.
//
// Restates src/sparse_attention.py:623-707 of the reference without ever
// materialising the per-row score tensor [B, H, M, NB]:
//   per-row score   S[r, blk] = sum_p sum_d Qcat_p[r, d] * planes[blk, p, d] * scaling
//                   (Quest: Qcat = (max(q,0), min(q,0)), planes = (Kmax, Kmin) —
//                   the two-matmul form of :638-642; mean: Qcat = (q, q) in fp16
//                   scaled by 2^qs per tile, planes = hi/lo of the block's fp32
//                   mean scaled by 2^e, both scales undone exactly on the fp32
//                   sum, :647-648);
//   tile max        T[t, blk] = max over the 64 rows of tile t (:655-656; rows
//                   past M are zero queries, as the reference's F.pad);
//   visibility      blocks past the tile's last row are -inf (:660-666);
//   forcing         T[0] = T[self] = FLT_MAX (:675-681);
//   top-k           k_slots best blocks ordered by (score desc, block asc) —
//                   torch.topk with its unspecified tie order made total (:697);
//   sigma           (s[k_base-1] - s[k_base]) / max(s[0] - s[k_base], 1e-6) in
//                   IEEE fp32 (correctly rounded division, denormals kept) (:703-707).
//
// Workgroup = W <= 8 consecutive (Q tile, query head) pairs of one (b, KV
// head g), tiles descending, one wavefront per pair (W chosen by the
// launcher from the LDS the row needs, so that two or more workgroups share
// a CU where they fit and one's top-k overlaps another's scoring; a
// workgroup may span two adjacent tiles, since the planes it stages are the
// KV head's).  The KV head's summary planes stream through LDS in
// chunks of CH blocks: chunk c + 1 is fetched into registers while chunk c
// is scored, then stored to the other of two buffers (one barrier per
// chunk), or, where only one buffer leaves room for a second workgroup on
// the CU, to the same buffer after a second barrier.  Each wave computes its 64 x CH score chunk on MFMA
// (A = its Q tile, with the Quest sign split done once, from registers;
// B = planes from LDS), max-pools it over rows in registers and appends CH
// tile scores to its LDS row.  The row then goes through a 4-pass 8-bit radix
// select for the k_slots-th best key, a ballot compaction of the winners
// (ties at the cut taken in block order) and a register bitonic sort.
//
// Dump mode (ugbsa_score_dump, the diagnostic of src/dump_block_scores.py:
// 137-171) runs the same scoring without the forcing, ranks k_slots =
// rho_k + 1 scores and writes the order-statistic gaps instead of kv_idx.
#pragma once

#include "common.h"
#include "launch.h"

namespace ugbsa {

constexpr int kSelWaves = 8;   // query heads (wavefronts) per workgroup, at most

struct SelectLds {
  int row_stride;      // elements per chunk row (P * D + 8 pad)
  int chunk_bytes;     // one chunk buffer
  int wave_bytes;
  int trow_off, hist_off, cand_off;  // within a wave's region
};

// Rows longer than this many blocks select by streaming (see stream_cap).
constexpr int kStreamBlocks = 4096;

// Candidate capacity of a streaming row: composite keys kept between
// shrinks (at least k_slots + one chunk; 4 * KP keeps shrinks rare).
__host__ __device__ constexpr int stream_cap(int KP) { return 4 * KP > 1024 ? 4 * KP : 1024; }

__host__ __device__ inline SelectLds select_lds(int P, int D, int NB, int KP, int CH,
                                                bool stream) {
  SelectLds s;
  s.row_stride = P * D + 8;
  s.chunk_bytes = CH * s.row_stride * 2;
  const int trow = (((stream ? CH : NB) * 4) + 15) / 16 * 16;
  s.trow_off = 0;
  s.hist_off = trow;
  s.cand_off = trow + 256 * 4;
  s.wave_bytes = s.cand_off + (stream ? stream_cap(KP) : KP) * 8;
  return s;
}

// Visible blocks whose keys the top-k keeps in registers (64 per lane step);
// longer rows run the same radix select on their LDS row.
constexpr int kRegKeys = 32;

// One radix-select step: hist holds 256 digit counts of the keys still in
// play; returns the digit of the remaining-th largest key and leaves in
// remaining its rank among the keys with that digit.
__device__ __forceinline__ int radix_digit(const uint32_t* hist, int lane, int& remaining,
                                           int& bin_count) {
  // lane L holds bins 255-4L .. 252-4L (descending digit order)
  uint32_t cnt[4], s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) { cnt[j] = hist[255 - 4 * lane - j]; s += cnt[j]; }
  uint32_t cg = wave_excl_scan(s, lane);   // keys in strictly greater digits
  int found = -1;
  uint32_t rem_new = 0, fcnt = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (found < 0 && cg < static_cast<uint32_t>(remaining) &&
        static_cast<uint32_t>(remaining) <= cg + cnt[j]) {
      found = 255 - 4 * lane - j;
      rem_new = remaining - cg;
      fcnt = cnt[j];
    }
    cg += cnt[j];
  }
  const uint64_t who = __ballot(found >= 0);
  const int src = __ffsll(static_cast<long long>(who)) - 1;
  remaining = __shfl(static_cast<int>(rem_new), src, 64);
  bin_count = __shfl(static_cast<int>(fcnt), src, 64);
  return __shfl(found, src, 64);
}

// Keeps the K best of the n composite keys (score key << 32 | ~block) in
// cand, in place and in cand order: a 4-pass radix select of the K-th
// largest score key tau, then a stable compaction of the keys above tau and
// the first (in cand order, i.e. lowest block) of those equal to it.
// Returns tau; n must exceed K.
__device__ inline uint32_t shrink_cand(uint64_t* cand, int n, int K, uint32_t* hist, int lane,
                                       uint64_t lt_mask) {
  uint32_t prefix = 0, pmask = 0;
  int remaining = K;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = lane; i < 256; i += 64) hist[i] = 0;
    wave_lds_sync();
    for (int i = lane; i < n; i += 64) {
      const uint32_t key = static_cast<uint32_t>(cand[i] >> 32);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    wave_lds_sync();
    int bin_count;
    const int digit = radix_digit(hist, lane, remaining, bin_count);
    prefix |= static_cast<uint32_t>(digit) << shift;
    pmask |= 0xFFu << shift;
    wave_lds_sync();
  }
  const int need_eq = remaining;
  int out = 0, eq_seen = 0;
  for (int base = 0; base < n; base += 64) {
    // every lane reads its key before any lane writes, and writes land
    // below base + 64, so the compaction can run in place
    const int i = base + lane;
    const uint64_t x = i < n ? cand[i] : 0ull;
    const uint32_t key = static_cast<uint32_t>(x >> 32);
    const bool gt = i < n && key > prefix;
    const bool eq = i < n && key == prefix;
    const uint64_t be = __ballot(eq);
    const bool keep = gt || (eq && eq_seen + __popcll(be & lt_mask) < need_eq);
    const uint64_t bk = __ballot(keep);
    if (keep) cand[out + __popcll(bk & lt_mask)] = x;
    out += __popcll(bk);
    eq_seen += __popcll(be);
  }
  wave_lds_sync();
  return prefix;
}

// Top-K of trow[0 .. n_vis) by (score desc, block asc) into cand[0 ..
// min(n_vis, K)) as composite keys (score key << 32 | ~block), unordered.
// The wave's LDS row, histogram and candidate buffer; wave-local.
template <int RK = kRegKeys>
__device__ __forceinline__ void select_to_cand(const float* trow, int n_vis, int K, uint32_t* hist,
                                               uint64_t* cand, int lane, uint64_t lt_mask) {
  if (n_vis > K) {
    // Radix select of the K-th largest key tau (8-bit digits from the most
    // significant), then the keys > tau and the first (K - #greater) keys
    // == tau in block order are compacted into cand.
    uint32_t prefix = 0, pmask = 0;
    int remaining = K;
    bool fast = false;
    if (n_vis <= 64 * RK) {
      // Rows of up to 64 * RK blocks: keys in registers.  The digits
      // start below the bits that every score except the two forced ones
      // shares (their AND / OR over the wavefront), so the first pass
      // spreads the scores over the bins instead of piling them into the
      // few that the exponent leaves.
      const int jmax = (n_vis + 63) / 64;
      uint32_t key[RK];
      uint32_t kand = 0xFFFFFFFFu, kor = 0u;
      static_for<RK>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        key[j] = 0u;
        if (j < jmax) {
          const int i = lane + 64 * j;
          if (i < n_vis) {
            key[j] = float_key(trow[i]);
            if (i != 0 && i != n_vis - 1) { kand &= key[j]; kor |= key[j]; }
          }
        }
      });
      kand = wave_and_u32(kand, lane);
      kor = wave_or_u32(kor, lane);
      const uint32_t diff = kand ^ kor;
      const int common = diff ? __clz(static_cast<int>(diff)) : 32;
      pmask = common ? (0xFFFFFFFFu << (32 - common)) : 0u;
      prefix = kand & pmask;
      // keys outside the common prefix, above or below its whole range: only
      // positions 0 and n_vis - 1 (n_vis > K >= 1, so two of them), which the
      // AND / OR leaves out — every other key shares the prefix by
      // construction — so their two keys decide the counts
      const uint32_t kf = float_key(trow[0]) & pmask;
      const uint32_t kl = float_key(trow[n_vis - 1]) & pmask;
      const int above = (kf > prefix ? 1 : 0) + (kl > prefix ? 1 : 0);
      const int below = (kf < prefix ? 1 : 0) + (kl < prefix ? 1 : 0);
      remaining = K - above;
      fast = remaining > 0 && remaining <= n_vis - above - below;
      if (fast) {
        for (int shift = 32 - common; shift > 0;) {
          const int d = shift < 8 ? shift : 8;
          shift -= d;
          const uint32_t dmask = (1u << d) - 1u;
          for (int i = lane; i < 256; i += 64) hist[i] = 0;
          wave_lds_sync();
          static_for<RK>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (j < jmax && lane + 64 * j < n_vis && (key[j] & pmask) == prefix)
              atomicAdd(&hist[(key[j] >> shift) & dmask], 1u);
          });
          wave_lds_sync();
          int bin_count;
          const int digit = radix_digit(hist, lane, remaining, bin_count);
          prefix |= static_cast<uint32_t>(digit) << shift;
          pmask |= dmask << shift;
          wave_lds_sync();
          // every key with this prefix is selected: the lower digits do
          // not matter (the sort below orders the selection exactly)
          if (remaining == bin_count) break;
        }
        const int need_eq = remaining;
        const int n_gt = K - need_eq;
        int cnt_gt = 0, cnt_eq = 0;
        static_for<RK>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          if (j < jmax) {
            const int i = lane + 64 * j;
            const uint32_t kp = key[j] & pmask;
            const bool gt = i < n_vis && kp > prefix;
            const bool eq = i < n_vis && kp == prefix;
            const uint64_t bg = __ballot(gt), be = __ballot(eq);
            const uint64_t comp = (static_cast<uint64_t>(key[j]) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
            if (gt) {
              const int pos = cnt_gt + __popcll(bg & lt_mask);
              if (pos < n_gt) cand[pos] = comp;
            }
            if (eq) {
              const int pos = cnt_eq + __popcll(be & lt_mask);
              if (pos < need_eq) cand[n_gt + pos] = comp;
            }
            cnt_gt += __popcll(bg);
            cnt_eq += __popcll(be);
          }
        });
      } else {
        prefix = 0;
        pmask = 0;
        remaining = K;
      }
    }
    if (!fast) {
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = lane; i < 256; i += 64) hist[i] = 0;
      wave_lds_sync();
      for (int i = lane; i < n_vis; i += 64) {
        const uint32_t key = float_key(trow[i]);
        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      wave_lds_sync();
      int bin_count;
      const int digit = radix_digit(hist, lane, remaining, bin_count);
      prefix |= static_cast<uint32_t>(digit) << shift;
      pmask |= 0xFFu << shift;
      wave_lds_sync();
    }
    const uint32_t tau = prefix;
    const int need_eq = remaining;
    const int n_gt = K - need_eq;
    int cnt_gt = 0, cnt_eq = 0;
    for (int base = 0; base < n_vis; base += 64) {
      const int i = base + lane;
      const uint32_t key = i < n_vis ? float_key(trow[i]) : 0u;
      const bool gt = i < n_vis && key > tau;
      const bool eq = i < n_vis && key == tau;
      const uint64_t bg = __ballot(gt), be = __ballot(eq);
      const uint64_t comp = (static_cast<uint64_t>(key) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
      if (gt) {
        const int pos = cnt_gt + __popcll(bg & lt_mask);
        if (pos < n_gt) cand[pos] = comp;
      }
      if (eq) {
        const int pos = cnt_eq + __popcll(be & lt_mask);
        if (pos < need_eq) cand[n_gt + pos] = comp;
      }
      cnt_gt += __popcll(bg);
      cnt_eq += __popcll(be);
    }
    }
  } else {
    for (int i = lane; i < n_vis; i += 64)
      cand[i] = (static_cast<uint64_t>(float_key(trow[i])) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
  }
}

// Loads cand[0 .. n_sel) into v (element e = lane + 64 r) and sorts it
// descending: a register bitonic sort over KP elements.
template <int KP>
__device__ __forceinline__ void sort_cand(const uint64_t* cand, int n_sel, int lane,
                                          uint64_t (&v)[KP / 64]) {
  constexpr int R = KP / 64;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int e = lane + 64 * r;
    v[r] = e < n_sel ? cand[e] : 0ull;
  }
  // bitonic sort, descending: stage (kk, j) compares element e with e ^ j,
  // across registers for j >= 64, across lanes (register shuffles) below
  constexpr int LOG_KP = KP == 64 ? 6 : KP == 128 ? 7 : KP == 256 ? 8 : 9;
  static_assert((1 << LOG_KP) == KP, "KP is a power of two");
  static_for<LOG_KP>([&](auto lk) {
    constexpr int kk = 2 << decltype(lk)::value;
    static_for<decltype(lk)::value + 1>([&](auto lj) {
      constexpr int j = (kk >> 1) >> decltype(lj)::value;
      uint64_t nv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int e = lane + 64 * r;
        uint64_t other;
        if constexpr (j >= 64) other = v[r ^ (j >> 6)];
        else other = xor_lanes_u64<j>(v[r], lane);
        const bool lower = (e & j) == 0;
        const bool desc = (e & kk) == 0;
        const bool keep_max = lower == desc;
        nv[r] = (keep_max == (v[r] > other)) ? v[r] : other;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) v[r] = nv[r];
    });
  });
}

// Score of rank e (0 = best) of a sorted v; -inf at ranks past n_sel.
template <int R>
__device__ __forceinline__ float sorted_value(const uint64_t (&v)[R], int e, int n_sel) {
  uint64_t x = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r == (e >> 6)) x = v[r];
  const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(x >> 32), e & 63, 64));
  return e < n_sel ? key_float(hi) : -INFINITY;
}

// Blocks per LDS chunk: 32 while a block's planes are at most 512 bytes, else 16.
__host__ __device__ constexpr int select_chunk(int P, int D) { return P * D <= 256 ? 32 : 16; }

// W: pairs (waves) per workgroup; wpb: workgroups per (b, KV head); nbuf:
// plane chunk buffers in LDS, 2 (double-buffered) or 1 (a second barrier
// per chunk), as the launcher sized the workgroup's LDS.
template <typename E, int D, bool QUEST, int KP, bool STREAM, bool ROWS>
__global__ __launch_bounds__(64 * kSelWaves) void select_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
    const uint16_t* __restrict__ planes, const float* __restrict__ bscale, int B, int Hk, int M,
    int N, int NB, int Qt, int grp,
    int W, int wpb, float scaling, int k_base, int k_slots, int want_sigma,
    int32_t* __restrict__ kv_idx, float* __restrict__ sigma, float* __restrict__ tile_score,
    const SelectAux aux, int nbuf) {
  constexpr int KS = D / 32;
  constexpr int R = KP / 64;
  constexpr int P = 2;                              // planes per block
  // MFMA format: Quest multiplies the input values; the mean planes are fp16
  using EM = std::conditional_t<QUEST, E, ElemF16>;
  constexpr int CH = select_chunk(P, D);
  constexpr int NT = CH / 16;                       // MFMA column tiles per chunk
  constexpr int PIECES = CH * P * D / 8;            // 16-byte pieces per chunk
  // pieces a thread prefetches into registers (enough for 4 or more waves;
  // smaller workgroups copy the rest when the chunk is stored)
  constexpr int STAGE = (PIECES + 255) / 256;
  // Quest multiplies max(q, 0) by the K-max plane and min(q, 0) by the
  // K-min plane.  The two signed copies of the Q tile are kept when they fit
  // (2 * 4 * KS fragments); at head_dim 256, and in the streaming rows that
  // hold extra state, only q is kept and the halves are formed per chunk.
  constexpr bool SPLIT_LATE = QUEST && (D > 128 || STREAM);
  constexpr int QSETS = QUEST && !SPLIT_LATE ? 2 : 1;
  extern __shared__ __align__(16) unsigned char smem[];
  const SelectLds L = select_lds(P, D, NB, KP, CH, STREAM);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, r16 = lane & 15;
  const int nthreads = blockDim.x;

  // The (tile, query head) pairs of one (b, KV head g), tiles descending,
  // run W to a workgroup (wpb workgroups per (b, g)), so a workgroup may
  // take the last heads of tile t and the first of tile t - 1: the planes it
  // stages are the KV head's, whichever tile reads them.  Workgroup i takes
  // pair block i / (B Hk) of (b, g) = i % (B Hk): all KV heads' heaviest
  // tiles first.  Pairs past the end of the range (the last block) idle.
  const int t_hi = ROWS ? aux.rows_t1 : Qt;
  const int pairs = (t_hi - (ROWS ? aux.rows_t0 : 0)) * grp;
  const int bg = blockIdx.x % (B * Hk);
  const int b = bg / Hk;
  const int g = bg % Hk;
  const int p0 = (blockIdx.x / (B * Hk)) * W;       // first pair of the workgroup
  const bool active = p0 + wave < pairs;
  const int pw = active ? p0 + wave : p0;
  const int t = t_hi - 1 - pw / grp;
  const int h = g * grp + pw % grp;
  const int t_first = t_hi - 1 - p0 / grp;          // the workgroup's largest tile
  const int H = Hk * grp;

  // chunk buffer i at smem + i * chunk_bytes (derived from smem each time, so
  // the compiler keeps LDS addressing for the operand reads)
  auto chunk_buf = [&](int i) -> uint16_t* {
    return reinterpret_cast<uint16_t*>(smem + i * L.chunk_bytes);
  };
  unsigned char* wreg = smem + nbuf * L.chunk_bytes + wave * L.wave_bytes;
  float* trow = reinterpret_cast<float*>(wreg + L.trow_off);
  uint32_t* hist = reinterpret_cast<uint32_t*>(wreg + L.hist_off);
  uint64_t* cand = reinterpret_cast<uint64_t*>(wreg + L.cand_off);

  const int last_row = min(t * kBlock + kBlock - 1, N - 1);
  const int n_vis = last_row / kBlock + 1;           // blocks 0 .. self(t)
  const int64_t row_id = (static_cast<int64_t>(b) * H + h) * Qt + t;
  float* ts = tile_score != nullptr ? tile_score + row_id * NB : nullptr;
  const int K = k_slots;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // streaming rows: candidates kept so far and the score key they all beat
  int cnt = 0;
  uint32_t cut = 0u;
  bool have_cut = false;

  // Q tile rows as MFMA A operands (zero rows past M, as F.pad in the
  // reference); Quest keeps (max(q, 0), min(q, 0)), which multiply the
  // K-max and K-min planes.
  bf16x8 qf[QSETS][4][KS];
  {
    const uint16_t* qb = q + b * sq_b + h * sq_h;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int row = t * kBlock + 16 * mt + r16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 x = (active && row < M) ? load_bf16x8(qb + row * sq_m + 32 * ks + 8 * g4)
                                             : zero_bf16x8();
        if constexpr (QUEST && !SPLIT_LATE) {
          qf[0][mt][ks] = bf16_pos(x);
          qf[1][mt][ks] = bf16_neg(x);
        } else {
          qf[0][mt][ks] = x;
        }
      }
    }
  }
  // mean: Q in fp16, scaled by 2^qs with max |q| 2^qs in [2^14, 2^15) over
  // the tile (exact for every element within 2^29 of the tile's largest);
  // tdesc = 2^-qs undoes it on the scores
  float tdesc = 1.f;
  if constexpr (!QUEST) tdesc = q_tile_to_f16<E, 4 * KS>(&qf[0][0][0], lane);

  const uint16_t* pl = planes + (static_cast<int64_t>(b) * Hk + g) * NB * P * D;
  // mean: 2^-e of each block of the KV head; the chunk's are loaded into
  // bsn one chunk ahead, with its planes
  const float* bs = QUEST ? nullptr : bscale + (static_cast<int64_t>(b) * Hk + g) * NB;
  float bsc[NT], bsn[NT];
  auto scale_load = [&](int c, float (&dst)[NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int blk = c * CH + 16 * nt + r16;
      dst[nt] = blk < NB ? bs[blk] : 0.f;
    }
  };
  constexpr int pieces_per_blk = P * D / 8;
  // chunks up to the workgroup's largest tile (a wave of the next tile
  // scores one block past its row, which its selection never reads)
  const int n_chunks = (min(t_first * kBlock + kBlock - 1, N - 1) / kBlock + CH) / CH;
  u32x4 stage[STAGE];
  // A chunk's blocks are contiguous, so piece pi of any chunk sits at byte
  // 16 pi from the chunk's start: each thread's offsets are fixed.  Pieces
  // past PIECES (a workgroup with more threads than a stage needs) get an
  // offset beyond every range.
  uint32_t voff[STAGE];
#pragma unroll
  for (int j = 0; j < STAGE; ++j) {
    const int pi = threadIdx.x + j * nthreads;
    voff[j] = pi < PIECES ? 16u * static_cast<uint32_t>(pi) : 0x80000000u;
  }
  // Chunk c through a buffer resource from the chunk's first block to block
  // NB: pieces past the last block read zeros (the F.pad rows of the
  // reference's summaries never reach a score), with no branch or clearing.
  auto fetch = [&](int c) {
    const int left = NB - c * CH;                     // >= 1 for every chunk fetched
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(pl + static_cast<int64_t>(c) * CH * P * D,
                  static_cast<uint32_t>(left) * (P * D * 2));
#pragma unroll
    for (int j = 0; j < STAGE; ++j)
      stage[j] = __builtin_bit_cast(u32x4, buffer_load_bf16x8(rs, voff[j], 0u));
  };
  auto store = [&](int buf, int c) {
#pragma unroll
    for (int j = 0; j < STAGE; ++j) {
      const int pi = threadIdx.x + j * nthreads;
      const int bl = pi / pieces_per_blk, off = pi % pieces_per_blk;
      if (pi < PIECES) *reinterpret_cast<u32x4*>(chunk_buf(buf) + bl * L.row_stride + off * 8) = stage[j];
    }
    for (int pi = threadIdx.x + STAGE * nthreads; pi < PIECES; pi += nthreads) {
      const int bl = pi / pieces_per_blk, off = pi % pieces_per_blk;
      const int blk = c * CH + bl;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (blk < NB) v = *reinterpret_cast<const u32x4*>(pl + static_cast<int64_t>(blk) * P * D + off * 8);
      *reinterpret_cast<u32x4*>(chunk_buf(buf) + bl * L.row_stride + off * 8) = v;
    }
  };
  const bool pos_scale = scaling >= 0.f;
  // +inf in a register the optimiser cannot see through (tile max-pool)
  float pinf = INFINITY;
  asm volatile("" : "+v"(pinf));

  fetch(0);
  if constexpr (!QUEST) scale_load(0, bsc);
  store(0, 0);
  __syncthreads();
  for (int c = 0; c < n_chunks; ++c) {
    const bool more = c + 1 < n_chunks;
    if (more) fetch(c + 1);
    if constexpr (!QUEST) {
      if (more) scale_load(c + 1, bsn);
    }
    if (active) {
      const uint16_t* chunk = chunk_buf(nbuf == 2 ? (c & 1) : 0);
      f32x4 acc[4][NT];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      // B fragments of step s = (p, ks) from LDS, requested two steps ahead
      // of their MFMAs (in program order, so that each step's reads are in
      // flight behind the two previous steps' 4 * NT MFMAs each instead of
      // waited for in full before them; one step ahead measured 2-3 %
      // slower at 128K with Quest planes, the same elsewhere)
      auto bload = [&](int s, bf16x8 (&dst)[NT]) {
        const int p = s / KS, ks = s % KS;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          dst[nt] = *reinterpret_cast<const bf16x8*>(chunk + (16 * nt + r16) * L.row_stride +
                                                     p * D + 32 * ks + 8 * g4);
      };
      bf16x8 bq[3][NT];
      bload(0, bq[0]);
      if constexpr (P * KS > 1) bload(1, bq[1]);
      static_for<P * KS>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        constexpr int p = s / KS, ks = s % KS;
        if constexpr (s + 2 < P * KS) bload(s + 2, bq[(s + 2) % 3]);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          bf16x8 a;
          if constexpr (SPLIT_LATE) {
            // the opaque copy keeps the split inside the chunk loop (hoisted,
            // both halves would stay live for the whole row)
            bf16x8 x = qf[0][mt][ks];
            asm volatile("" : "+v"(x));
            a = p == 0 ? bf16_pos(x) : bf16_neg(x);
          } else {
            a = qf[QSETS == 2 ? p : 0][mt][ks];
          }
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = EM::mfma(a, bq[s % 3][nt], acc[mt][nt]);
        }
        // keep each step's reads ahead of the previous step's MFMAs (the
        // scheduler would otherwise pair two steps' reads and wait on them)
        __builtin_amdgcn_sched_barrier(0);
      });
      // the exact factor from the MFMA sums to the scores of column nt (1
      // for Quest; a product of two powers of two for the mean)
      float cs[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) cs[nt] = QUEST ? 1.f : bsc[nt] * tdesc;
      if constexpr (ROWS) {
        // per-row scores (the v1 selector's input): fl(raw * scaling), -inf
        // past the tile's visible blocks, rows past M skipped
        const int64_t nrows = 64 * static_cast<int64_t>(aux.rows_t1 - aux.rows_t0);
        float* rs = aux.row_scores + (static_cast<int64_t>(b) * H + h) * nrows * NB +
                    static_cast<int64_t>(t - aux.rows_t0) * 64 * NB;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int r = 16 * mt + 4 * g4 + i;
              const int blk = c * CH + 16 * nt + r16;
              if (t * kBlock + r < M && blk < NB)
                rs[static_cast<int64_t>(r) * NB + blk] =
                    blk < n_vis ? (QUEST ? acc[mt][nt][i] : acc[mt][nt][i] * cs[nt]) * scaling
                                : -INFINITY;
            }
      } else {
        // tile max over the 64 rows of (score * scaling): the max (min for a
        // negative scaling) of the raw sums, scaled once — fl(x * s) is
        // monotone in x, so this is the max of the scaled scores exactly.
        // (v_med3 with an opaque +-inf bound: max / min without the
        // canonicalising copies fmaxf / fminf of MFMA results get)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float bound = pos_scale ? pinf : -pinf;
          float mx = acc[0][nt][0];
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = __builtin_amdgcn_fmed3f(mx, acc[mt][nt][i], bound);
          mx = quad_rows_med3(mx, bound);
          const int blk = c * CH + 16 * nt + r16;
          if constexpr (!QUEST) mx *= cs[nt];
          if (g4 == nt % 4 && blk < NB) trow[STREAM ? 16 * nt + r16 : blk] = mx * scaling;
        }
        if constexpr (STREAM) {
          // Append the chunk's visible scores that beat the cut, in block
          // order (forcing applied); shrink to the K best before the buffer
          // could overflow.  The K best of the row are then always among
          // the candidates: a later block that ties the cut ranks below every
          // kept key of that score (higher block index).
          wave_lds_sync();
          const int blk = c * CH + lane;
          const bool ok = lane < CH && blk < n_vis;
          float sc = ok ? trow[lane] : 0.f;
          if (!aux.dump && (blk == 0 || blk == n_vis - 1)) sc = kFMax;
          if (ok && ts != nullptr) ts[blk] = sc;
          const uint32_t key = float_key(sc);
          const bool take = ok && (!have_cut || key > cut);
          const uint64_t bal = __ballot(take);
          if (take)
            cand[cnt + __popcll(bal & lt_mask)] =
                (static_cast<uint64_t>(key) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(blk));
          cnt += __popcll(bal);
          if (cnt > stream_cap(KP) - CH) {
            wave_lds_sync();
            cut = shrink_cand(cand, cnt, K, hist, lane, lt_mask);
            cnt = K;
            have_cut = true;
          }
        }
      }
    }
    if (nbuf == 1) __syncthreads();       // every wave is done with the one buffer
    if (more) store(nbuf == 2 ? ((c + 1) & 1) : 0, c + 1);
    if constexpr (!QUEST) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bsc[nt] = bsn[nt];
    }
    __syncthreads();
  }
  if (!active) return;   // no workgroup barrier follows
  if constexpr (ROWS) {
    // blocks past the last computed chunk: -inf
    const int64_t nrows = 64 * static_cast<int64_t>(aux.rows_t1 - aux.rows_t0);
    float* rs = aux.row_scores + (static_cast<int64_t>(b) * H + h) * nrows * NB +
                static_cast<int64_t>(t - aux.rows_t0) * 64 * NB;
    const int r_end = min(kBlock, M - t * kBlock);
    for (int r = 0; r < r_end; ++r)
      for (int blk = n_chunks * CH + lane; blk < NB; blk += 64) rs[static_cast<int64_t>(r) * NB + blk] = -INFINITY;
    return;
  }
  wave_lds_sync();
  const int n_sel = min(n_vis, K);
  if constexpr (STREAM) {
    if (ts != nullptr)
      for (int i = n_vis + lane; i < NB; i += 64) ts[i] = -INFINITY;
    if (cnt > K) shrink_cand(cand, cnt, K, hist, lane, lt_mask);
  } else {
    if (lane == 0 && !aux.dump) {
      trow[0] = kFMax;
      trow[n_vis - 1] = kFMax;
    }
    wave_lds_sync();
    if (ts != nullptr)
      for (int i = lane; i < NB; i += 64) ts[i] = i < n_vis ? trow[i] : -INFINITY;
    // register keys sized to the row (8, 16 or 32 per lane): the key loops
    // are unrolled over the slots, so a short row runs far fewer of them
    // (select at c2 0.175 -> 0.161 ms, c3 1.77 -> 1.72, c4 0.741 -> 0.705;
    // 4 per lane for rows of up to 256 blocks gains nothing more)
    if (n_vis <= 64 * 8) select_to_cand<8>(trow, n_vis, K, hist, cand, lane, lt_mask);
    else if (n_vis <= 64 * 16) select_to_cand<16>(trow, n_vis, K, hist, cand, lane, lt_mask);
    else select_to_cand<kRegKeys>(trow, n_vis, K, hist, cand, lane, lt_mask);
  }
  wave_lds_sync();

  uint64_t v[R];
  sort_cand<KP>(cand, n_sel, lane, v);

  if (kv_idx != nullptr) {
    int32_t* out = kv_idx + row_id * K;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = lane + 64 * r;
      if (e < K)
        out[e] = e < n_sel ? static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(v[r])) : e;
    }
  }

  auto val_at = [&](int e) -> float { return sorted_value<R>(v, e, n_sel); };
  if (aux.dump) {
    // src/dump_block_scores.py:161-171, on the unforced scores: g, r
    // (clamp(min=1e-9)), sigma = clamp(g / r, 0, 2) and g_rho, NaN kept
    // where ranks past the visible blocks meet (-inf - -inf)
    const float s0 = val_at(0);
    const float skm1 = val_at(aux.k_b - 1), sk = val_at(aux.k_b);
    const float srm1 = val_at(aux.rho_k - 1), srk = val_at(aux.rho_k);
    const float gg = skm1 - sk;
    float rr = s0 - sk;
    if (rr < 1e-9f) rr = 1e-9f;
    float sg = gg / rr;
    if (sg < 0.f) sg = 0.f;
    if (sg > 2.f) sg = 2.f;
    if (lane == 0) {
      aux.g[row_id] = gg;
      aux.r[row_id] = rr;
      aux.sigma[row_id] = sg;
      aux.g_rho[row_id] = srm1 - srk;
      if (b == 0 && h == 0) aux.valid[t] = n_vis > aux.rho_k ? 1 : 0;
    }
    return;
  }

  if (want_sigma) {
    const float s_top = val_at(0);
    const float a = val_at(k_base - 1);
    const float cth = val_at(k_base);
    float spread = s_top - cth;
    if (spread < 1e-6f) spread = 1e-6f;     // clamp(min=1e-6); NaN stays NaN
    const float sg = (a - cth) / spread;
    if (lane == 0) sigma[row_id] = sg;
  }
}

template <typename E, int D, bool QUEST, int KP, bool STREAM, bool ROWS = false>
static hipError_t launch_select_t(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                  const uint16_t* planes, int B, int H, int Hk, int M, int N,
                                  float scaling, int k_base, int k_slots, int want_sigma,
                                  int32_t* kv_idx, float* sigma, float* tile_score,
                                  const SelectAux& aux, hipStream_t stream) {
  const int NB = (N + kBlock - 1) / kBlock;
  const int Qt = (M + kBlock - 1) / kBlock;
  const int grp = H / Hk;
  const SelectLds L = select_lds(2, D, NB, KP, select_chunk(2, D), STREAM);
  constexpr int kLdsMax = 160 * 1024;
  // W (tile, head) pairs per workgroup, one wavefront each: the W that
  // keeps the most wavefronts on a CU, given its LDS and at most 8 resident
  // waves (about 230 VGPRs each), counting 10 % more when two or more
  // workgroups share the CU (one's top-k then overlaps another's scoring);
  // ties go to the larger W, which stages each plane chunk for more pairs,
  // and to two chunk buffers over one (one fewer barrier per chunk; one
  // buffer wins where it alone fits a second workgroup, as at head_dim 256
  // with three planes: 2.55 -> 2.33 ms at 128K keys).  W < 4 counts half:
  // such workgroups cannot prefetch a whole chunk into registers (they are
  // only chosen when a long key range leaves no room in LDS for more waves).
  int W = 0, nbuf = 2;
  double best = -1.0;
  for (int nb = 2; nb >= 1; --nb)
    for (int w = 1; w <= kSelWaves; ++w) {
      const size_t lds_w = nb * static_cast<size_t>(L.chunk_bytes) + static_cast<size_t>(w) * L.wave_bytes;
      if (lds_w > static_cast<size_t>(kLdsMax)) break;
      int per_cu = static_cast<int>(kLdsMax / lds_w);
      if (per_cu > 8 / w) per_cu = 8 / w;
      const double active = per_cu * static_cast<double>(w) * (per_cu >= 2 ? 1.1 : 1.0) *
                            (w < 4 ? 0.5 : 1.0);
      if (active > best || (active == best && nb == nbuf)) { best = active; W = w; nbuf = nb; }
    }
  if (W == 0) return hipErrorInvalidConfiguration;
  const size_t lds = nbuf * static_cast<size_t>(L.chunk_bytes) + static_cast<size_t>(W) * L.wave_bytes;
  const int tiles = ROWS ? aux.rows_t1 - aux.rows_t0 : Qt;
  const int wpb = (tiles * grp + W - 1) / W;        // workgroups per (b, KV head)
  const int64_t wgs = static_cast<int64_t>(B) * Hk * wpb;
  auto kern = select_kernel<E, D, QUEST, KP, STREAM, ROWS>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(lds));
  if (e != hipSuccess) return e;
  kern<<<dim3(static_cast<unsigned>(wgs)), 64 * W, lds, stream>>>(
      q, sq_b, sq_h, sq_m, planes, QUEST ? nullptr : mean_descale(planes, B, Hk, NB, D), B, Hk,
      M, N, NB, Qt, grp, W, wpb, scaling, k_base,
      k_slots, want_sigma, kv_idx, sigma, tile_score, aux, nbuf);
  return hipGetLastError();
}

template <typename E, int D, bool QUEST>
static hipError_t launch_select_kp(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                                   const uint16_t* planes, int B, int H, int Hk, int M, int N,
                                   float scaling, int k_base, int k_slots, int want_sigma,
                                   int32_t* kv_idx, float* sigma, float* tile_score,
                                   const SelectAux& aux, hipStream_t stream) {
  // per-row scores only: the smallest LDS layout (no row, no top-k)
  if (aux.row_scores != nullptr)
    return launch_select_t<E, D, QUEST, 64, true, true>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N,
                                                 scaling, 1, 1, 0, nullptr, nullptr, nullptr, aux,
                                                 stream);
  // rows of more than kStreamBlocks blocks stream their candidates, so that
  // LDS per wave does not grow with the context
  const bool stream_rows = (N + kBlock - 1) / kBlock > kStreamBlocks;
#define UGBSA_SEL(KP_)                                                                      \
  return stream_rows                                                                        \
             ? launch_select_t<E, D, QUEST, KP_, true>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, \
                                                scaling, k_base, k_slots, want_sigma, kv_idx,  \
                                                sigma, tile_score, aux, stream)                 \
             : launch_select_t<E, D, QUEST, KP_, false>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N,  \
                                                 scaling, k_base, k_slots, want_sigma, kv_idx, \
                                                 sigma, tile_score, aux, stream)
  if (k_slots <= 64) UGBSA_SEL(64);
  if (k_slots <= 128) UGBSA_SEL(128);
  if (k_slots <= 256) UGBSA_SEL(256);
  if (k_slots <= 512) UGBSA_SEL(512);
#undef UGBSA_SEL
  return hipErrorInvalidValue;
}

// The selection kernels of one element format (D and backbone dispatched here).
template <typename E>
hipError_t launch_select_e(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                         const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                         int mode, float scaling, int k_base, int k_slots, int want_sigma,
                         int32_t* kv_idx, float* sigma, float* tile_score,
                         hipStream_t stream, const SelectAux* aux) {
  const SelectAux off{};
  const SelectAux& dm = aux != nullptr ? *aux : off;
#define UGBSA_SELD(D_, Q_)                                                                 \
  return launch_select_kp<E, D_, Q_>(q, sq_b, sq_h, sq_m, planes, B, H, Hk, M, N, scaling,    \
                                  k_base, k_slots, want_sigma, kv_idx, sigma, tile_score,  \
                                  dm, stream)
  const bool quest = mode == kModeQuest;
  if (D == 64) { if (quest) UGBSA_SELD(64, true); else UGBSA_SELD(64, false); }
  if (D == 128) { if (quest) UGBSA_SELD(128, true); else UGBSA_SELD(128, false); }
  if (D == 256) { if (quest) UGBSA_SELD(256, true); else UGBSA_SELD(256, false); }
#undef UGBSA_SELD
  return hipErrorInvalidValue;
}

// fp16 instances (select_f16.hip, a compile unit of their own).
hipError_t launch_select_f16(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_m,
                             const uint16_t* planes, int B, int H, int Hk, int M, int N, int D,
                             int mode, float scaling, int k_base, int k_slots, int want_sigma,
                             int32_t* kv_idx, float* sigma, float* tile_score,
                             hipStream_t stream, const SelectAux* aux);

}  // namespace ugbsa
