// Shared device helpers for the gfx950 (CDNA4) sparse-prefill kernels.
//
// Conventions used by every kernel in this library:
//  * a wavefront is 64 lanes; lane = 16 * g4 + r16 (g4 = lane >> 4, r16 = lane & 15);
//  * MFMA v_mfma_f32_16x16x32_bf16: lane (r16, g4) supplies row r16 of A and
//    column r16 of B, each with 8 consecutive bf16 of the 32-long contraction
//    (slots 8*g4 .. 8*g4+7); it receives C[4*g4 + i][r16], i = 0..3.  Any
//    consistent relabelling of the contraction slots between A and B gives the
//    same product, which the kernels use to permute keys freely;
//  * 16-bit tensors (bf16 or fp16, one format per call: ElemBf16 / ElemF16
//    below) are read with 16-byte vector loads, so the innermost (D) stride
//    must be 1 and row strides multiples of 8 elements.  In registers and
//    LDS eight such elements travel as a bf16x8 whatever their format; the
//    format's MFMA and conversions interpret them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>


namespace ugbsa {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short i16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

constexpr int kWave = 64;
constexpr int kBlock = 64;          // tokens per KV block (reference BLOCK)
constexpr float kFMax = 3.40282346638528859812e+38f;
constexpr float kLog2e = 1.44269504088896340736f;
// Online softmax with a lazy offset: the exp2 offset of a row only moves when
// the row max exceeds it by more than this (log2 units), so P <= 2^8 and the
// O rescale is skipped on most blocks; O / l does not depend on the offset.
constexpr float kLazyLog2 = 8.0f;

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Global-memory pointers with a wave-uniform (SGPR) base: 16-byte slab s of
// a run of 1 KiB slabs at base is read at base + 4 KiB * (s / 4) (a scalar
// add) + lane_b + 1 KiB * (s % 4) (the instruction's offset field, which
// holds less than 4 KiB), so every load takes the SGPR-base form with one
// 32-bit lane offset instead of a 64-bit address per lane in VGPRs.
typedef const __attribute__((address_space(1))) char gchar;
typedef const __attribute__((address_space(1))) bf16x8 gbf16x8;
__device__ __forceinline__ gchar* uniform_gptr(gchar* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return reinterpret_cast<gchar*>((static_cast<uint64_t>(hi) << 32) | lo);
}
// Callers in loops refresh lane_b once per iteration with an empty volatile
// asm: a 64-bit copy of it hoisted out of the loop would hide the 32-bit
// offset that the SGPR-base form needs.
__device__ __forceinline__ bf16x8 load_slab(gchar* base, uint32_t lane_b, int s) {
  gchar* b4 = uniform_gptr(base + (s / 4) * 4096);
  return *reinterpret_cast<gbf16x8*>(b4 + (lane_b + static_cast<uint32_t>(s % 4) * 1024u));
}

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ bf16x8 zero_bf16x8() {
  i16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  return __builtin_bit_cast(bf16x8, z);
}

// max(x, 0) / min(x, 0) of eight bf16 values by sign masking (exact).
__device__ __forceinline__ bf16x8 bf16_pos(bf16x8 x) {
  i16x8 v = __builtin_bit_cast(i16x8, x);
  i16x8 s = v >> 15;                 // all ones where negative
  return __builtin_bit_cast(bf16x8, v & ~s);
}
__device__ __forceinline__ bf16x8 bf16_neg(bf16x8 x) {
  i16x8 v = __builtin_bit_cast(i16x8, x);
  i16x8 s = v >> 15;
  return __builtin_bit_cast(bf16x8, v & s);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (inputs here are finite).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 pairs -> bf16 with v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  const bf16x2 h = __builtin_convertvector(f32x2{a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Element formats of the 16-bit tensors (Q, K, V, the Quest summary planes
// and the attention output of one call share one; the mean summary planes
// are fp16 for both).  Products of two 16-bit values are exact in fp32 for
// both, so the fp32-accumulated scores and S = Q.K^T follow the same
// arithmetic in either format.
struct ElemBf16 {
  static constexpr int code = 0;
  __device__ static __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // round-to-nearest-even pair (lo = a)
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
  __device__ static __forceinline__ float to_f32(uint32_t h) { return __uint_as_float(h << 16); }
  __device__ static __forceinline__ uint16_t from_f32(float f) { return f32_to_bf16(f); }
};
struct ElemF16 {
  static constexpr int code = 1;
  __device__ static __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  __device__ static __forceinline__ float to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xFFFFu)));
  }
  __device__ static __forceinline__ uint16_t from_f32(float f) {
    return static_cast<uint16_t>(pack2(f, 0.f) & 0xFFFFu);
  }
};

// Two MFMAs accumulating in AGPRs, c0 += a0 . b0 and c1 += a1 . b1 (the
// accumulators never leave the AGPR file).  Written as inline assembly
// because the compiler, built with MFMA results in VGPRs, would otherwise
// place every accumulator there; its hazard recognizer does not look inside
// the asm, so the wait states are the caller's: a VALU write of an operand
// (A, B, or the accumulator after v_accvgpr_write) needs two before an MFMA
// reads it, and agpr_drain() gives the ones a VALU read of the results needs
// after the last MFMA.  The pair itself carries no s_nop: in the attention
// loop its operands are V^T fragments from memory, P formed a phase earlier
// and accumulators only these MFMAs write (a blanket s_nop 1 per pair cost
// 0.6 % at head_dim 256); tests/test_isa_hazards.py checks the emitted code
// for a VALU write of an operand within two wait states of the MFMA.
template <typename E>
__device__ __forceinline__ void mfma16x16x32_agpr2(f32x4& c0, bf16x8 a0, bf16x8 b0, f32x4& c1,
                                                   bf16x8 a1, bf16x8 b1) {
  if constexpr (E::code == ElemF16::code) {
    asm volatile(
        "v_mfma_f32_16x16x32_f16 %0, %2, %3, %0\n\t"
        "v_mfma_f32_16x16x32_f16 %1, %4, %5, %1"
        : "+a"(c0), "+a"(c1)
        : "v"(a0), "v"(b0), "v"(a1), "v"(b1));
  } else {
    asm volatile(
        "v_mfma_f32_16x16x32_bf16 %0, %2, %3, %0\n\t"
        "v_mfma_f32_16x16x32_bf16 %1, %4, %5, %1"
        : "+a"(c0), "+a"(c1)
        : "v"(a0), "v"(b0), "v"(a1), "v"(b1));
  }
}
// Wait states between the last MFMA writing AGPR accumulators and any
// other access to them (the compiler waits 8 after a 16x16x32 bf16 MFMA;
// 24 here).  Callers pin the accumulators after it ("+a" on an empty asm)
// so that no read of them is scheduled above it.
__device__ __forceinline__ void agpr_drain() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
}

__device__ __forceinline__ bf16x8 pack_bf16x8(const float* f) {
  u32x4 w;
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = cvt_pk_bf16(f[2 * j], f[2 * j + 1]);
  return __builtin_bit_cast(bf16x8, w);
}

// Raw buffer resource over [base, base + bytes): loads at byte offsets
// outside the range return zeros (no fault, no branch).  Word 3 = 0x00020000
// is the untyped raw-buffer configuration of gfx9-family parts.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}
// 16 bytes at (voffset + soffset) of a raw buffer.
__device__ __forceinline__ bf16x8 buffer_load_bf16x8(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                                    uint32_t soffset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voffset),
                                                        static_cast<int>(soffset), 0);
  return __builtin_bit_cast(bf16x8, v);
}

typedef __attribute__((address_space(3))) void lds_void;

// Asynchronous 16-byte-per-lane copy of a raw buffer into LDS: lane L's
// 16 bytes land at lds + 16 * L.  Completion is tracked with vmcnt; the
// compiler waits on the destination object before LDS reads of it.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds,
                                                  uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(lds), 16,
                                           static_cast<int>(voffset), static_cast<int>(soffset),
                                           0, 0);
}

// s_waitcnt lgkmcnt(0): every LDS read of this wave has returned.
__device__ __forceinline__ void wait_lds_reads() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Monotone uint32 key of an fp32 value (larger float -> larger key); NaN is
// mapped above +inf, matching torch.topk / kthvalue's NaN-is-largest order.
__device__ __forceinline__ uint32_t float_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (x != x) return 0xFFFFFFFFu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  if (k == 0xFFFFFFFFu) return __uint_as_float(0x7FC00000u);
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = 0 .. N - 1,
// so every index the body derives from I is a constant expression (array
// subscripts stay in registers whatever the loop body's size).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Cross-lane helpers within one wavefront.
__device__ __forceinline__ float shfl_xor_f(float v, int m) {
  return __shfl_xor(v, m, kWave);
}
__device__ __forceinline__ uint32_t shfl_xor_u(uint32_t v, int m) {
  return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m, kWave));
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = shfl_xor_u(static_cast<uint32_t>(v), m);
  uint32_t hi = shfl_xor_u(static_cast<uint32_t>(v >> 32), m);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Max / sum over the four lanes r, r + 16, r + 32, r + 48 (every lane gets
// the result).  v_permlane16_swap / v_permlane32_swap exchange 16-lane rows
// in the VALU, with no LDS round trip: swapping x with itself leaves rows
// (0, 0, 2, 2) in one half of the pair and (1, 1, 3, 3) in the other, so the
// element-wise op of the pair is the xor-16 reduction (likewise xor-32).
__device__ __forceinline__ float quad_rows_max(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// quad_rows_max with v_med3_f32(a, b, bound): bound = +inf gives max(a, b),
// -inf min(a, b), without the canonicalising copy IEEE mode puts before each
// fmaxf / fminf of an MFMA result.  bound must sit in a register the
// optimiser cannot see through (an empty asm on it), or the med3 folds back
// into fmaxf / fminf.
__device__ __forceinline__ float quad_rows_med3(float v, float bound) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __builtin_amdgcn_fmed3f(__uint_as_float(a[0]), __uint_as_float(a[1]), bound);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __builtin_amdgcn_fmed3f(__uint_as_float(b[0]), __uint_as_float(b[1]), bound);
}
__device__ __forceinline__ float quad_rows_sum(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// x of lane (lane ^ M) for a compile-time M, in VALU registers (no LDS
// crossbar): quad_perm for 1 and 2, row_ror 12 / 4 (lane gets lane + 4 /
// lane - 4 within its 16-lane row) for 4, row_ror 8 for 8, and the halves of
// v_permlane16_swap / v_permlane32_swap of x with itself (rows (0, 0, 2, 2) /
// (1, 1, 3, 3), halves (0, 0) / (1, 1)) for 16 and 32.
template <int M>
__device__ __forceinline__ uint32_t xor_lanes(uint32_t x, int lane) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane mask");
  const int v = static_cast<int>(x);
  if constexpr (M == 1) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));
  } else if constexpr (M == 2) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));
  } else if constexpr (M == 4) {
    const int down = __builtin_amdgcn_update_dpp(v, v, 0x124, 0xF, 0xF, false);
    const int up = __builtin_amdgcn_update_dpp(v, v, 0x12C, 0xF, 0xF, false);
    return static_cast<uint32_t>((lane & 4) ? down : up);
  } else if constexpr (M == 8) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false));
  } else if constexpr (M == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? p[0] : p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? p[0] : p[1];
  }
}
template <int M>
__device__ __forceinline__ uint64_t xor_lanes_u64(uint64_t x, int lane) {
  const uint32_t lo = xor_lanes<M>(static_cast<uint32_t>(x), lane);
  const uint32_t hi = xor_lanes<M>(static_cast<uint32_t>(x >> 32), lane);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Bitwise AND / OR across the wavefront (every lane gets the result).
__device__ __forceinline__ uint32_t wave_and_u32(uint32_t x, int lane) {
  x &= xor_lanes<32>(x, lane);
  x &= xor_lanes<16>(x, lane);
  x &= xor_lanes<8>(x, lane);
  x &= xor_lanes<4>(x, lane);
  x &= xor_lanes<2>(x, lane);
  return x & xor_lanes<1>(x, lane);
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t x, int lane) {
  x |= xor_lanes<32>(x, lane);
  x |= xor_lanes<16>(x, lane);
  x |= xor_lanes<8>(x, lane);
  x |= xor_lanes<4>(x, lane);
  x |= xor_lanes<2>(x, lane);
  return x | xor_lanes<1>(x, lane);
}

// Exclusive prefix sum across the wavefront.
__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t x, int lane) {
  uint32_t incl = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), off, 64));
    if (lane >= off) incl += y;
  }
  return incl - x;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x, int lane) {
  x = max(x, xor_lanes<32>(x, lane));
  x = max(x, xor_lanes<16>(x, lane));
  x = max(x, xor_lanes<8>(x, lane));
  x = max(x, xor_lanes<4>(x, lane));
  x = max(x, xor_lanes<2>(x, lane));
  return max(x, xor_lanes<1>(x, lane));
}

// The mean summary planes of kernel 1 ([B, Hk, NB, 2, D] fp16 hi / lo of
// each block's fp32 mean scaled by 2^e) are followed by the blocks' 2^-e,
// [B, Hk, NB] fp32.
__host__ __device__ inline const float* mean_descale(const uint16_t* planes, int B, int Hk, int NB,
                                                     int D) {
  return reinterpret_cast<const float*>(planes + static_cast<int64_t>(B) * Hk * NB * 2 * D);
}

// NF fragments of a Q tile (format E) to fp16 in place, scaled by 2^qs with
// qs chosen over the wavefront from the exponent field of the largest
// magnitude so that max |q| 2^qs lies in [2^14, 2^15) (qs = 0 for an all-zero
// tile).  Exact for every element within 2^29 of the largest: fp16 holds the
// 8 (bf16) or 11 (fp16) significant bits, and its normal range spans 2^-14 ..
// 2^15.  Returns 2^-qs, which undoes the scaling on a product exactly.
template <typename E, int NF>
__device__ __forceinline__ float q_tile_to_f16(bf16x8* f, int lane) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 mv = {0, 0};
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    const u32x4 w = __builtin_bit_cast(u32x4, f[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      mv = __builtin_elementwise_max(mv, __builtin_bit_cast(u16x2, w[j] & 0x7FFF7FFFu));
  }
  const uint32_t m = wave_max_u32(max(static_cast<uint32_t>(mv[0]), static_cast<uint32_t>(mv[1])), lane);
  constexpr bool kF16 = E::code == 1;
  const int qs = m == 0u ? 0 : (kF16 ? 29 - static_cast<int>(m >> 10) : 141 - static_cast<int>(m >> 7));
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    u32x4 w = __builtin_bit_cast(u32x4, f[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = ldexpf(E::to_f32(w[j] & 0xFFFFu), qs);
      const float b = ldexpf(E::to_f32(w[j] >> 16), qs);
      w[j] = ElemF16::pack2(a, b);
    }
    f[i] = __builtin_bit_cast(bf16x8, w);
  }
  return ldexpf(1.0f, -qs);
}

// Order LDS traffic of one wavefront against itself (no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace ugbsa
