// Shared device helpers for the GDN-2 HIP kernels (gfx950 / CDNA4).
//
// Numerics mirror the reference's precision helpers (atomic_gdn2/precision.py:8-52):
//   * sanitize(x, c)  = clip(x, -c, c) with NaN -> 0            (precision.py:51-52)
//   * exp_nonpos(x)   = exp(min(x, 0))                            (precision.py:41-44)
//   * dot modes       : highest = fp32 MFMA, bf16x3 = hi*hi + hi*lo + lo*hi on bf16 MFMA,
//                       default = one bf16 MFMA pass              (precision.py:8-31)
//
// MFMA tiles are 16x16 on wave64.  For v_mfma_f32_16x16x4_f32 lane l supplies A[l%16][l/16]
// and B[l/16][l%16]; for v_mfma_f32_16x16x16_bf16 lane l supplies A[l%16][4*(l/16)+e] and
// B[4*(l/16)+e][l%16], e = 0..3.  The 4 accumulator values of lane l are the outputs at
// row 4*(l/16)+r, column l%16, r = 0..3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace gdn2 {

constexpr int T = 64;        // chunk length (cfg.bt) supported by the kernels
constexpr int WAVE = 64;

enum DotMode : int { DOT_HIGHEST = 0, DOT_BF16X3 = 1, DOT_DEFAULT = 2 };
enum DiagMode : int { DIAG_BTL = 0, DIAG_LEAN = 1 };

typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
// Wave index as a provably wave-uniform value (SGPR): branches on it stay scalar, so no
// exec-mask merge (and no accumulator copy at such a merge) lands inside an MFMA chain.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE); }

// clamp as one v_med3_f32 (exact for every non-NaN x), NaN selected to 0
__device__ __forceinline__ float sanitize(float x, float c) {
  return x != x ? 0.f : __builtin_amdgcn_fmed3f(x, -c, c);
}

// e^x as one hardware 2^y (v_exp_f32) of y = x log2(e): the rounding of y gives a relative
// error of about |x| 6e-8 (<= 1.2e-6 for |x| <= 20, the gate range of the domain), against
// ~10 instructions for a range-reduced expf.  Used for every rescaling factor: the score
// legs and the element-wise gates.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// min(x, 0) and clip(x, lo, hi) with NaN kept, as jnp.minimum / jnp.clip do (fminf / fmaxf
// would return the other operand): IEEE 754-2019 minimum / maximum, one v_minimum3_f32 /
// v_maximum3_f32 each on gfx950.  A NaN gate therefore gives a NaN factor, which the next
// sanitize point turns into 0, exactly as in the reference.
__device__ __forceinline__ float min0(float x) { return __builtin_elementwise_minimum(x, 0.f); }
__device__ __forceinline__ float clip_nan(float x, float lo, float hi) {
  return __builtin_elementwise_minimum(__builtin_elementwise_maximum(x, lo), hi);
}

__device__ __forceinline__ float exp_nonpos(float x) { return fast_exp(min0(x)); }

// One element of the inter-chunk state update h = san(h e^gamma + (Kg^T v_new)), gamma <= 0
// (fwd/cd_slim.py:28-29).  The forward scan and the backward's state recompute both call this,
// so a recomputed state equals the forward's bit for bit.
__device__ __forceinline__ float state_update(float h, float gamma, float kv, float clip) {
  return sanitize(fmaf(h, exp_nonpos(gamma), kv), clip);
}

// ---- bfloat16 helpers: round-to-nearest-even (NaN stays NaN) --------------------------
// Two floats to two bfloat16, packed a | b << 16, by one v_cvt_pk_bf16_f32.
typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 b2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pack(float a, float b) {
  const f2v f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, b2v));
}
__device__ __forceinline__ uint32_t bf16_bits(float x) { return bf16_pack(x, 0.f) & 0xffffu; }
__device__ __forceinline__ float bf16_val(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf16_round(float x) { return bf16_val(bf16_bits(x)); }

// ---- strided operand views ----------------------------------------------------------
// at(r, c) = mul * p[r*sr + c*sc].  A operands are read as at(i, k), B operands as at(k, j).
struct View {
  const float* p;
  int sr, sc;
  float mul;
  __device__ __forceinline__ float at(int r, int c) const { return mul * p[r * sr + c * sc]; }
  __device__ __forceinline__ View shift(int dr, int dc) const {
    return View{p + dr * sr + dc * sc, sr, sc, mul};
  }
};
__device__ __forceinline__ View rm(const float* p, int ld, float mul = 1.f) { return View{p, ld, 1, mul}; }
__device__ __forceinline__ View tr(const float* p, int ld, float mul = 1.f) { return View{p, 1, ld, mul}; }

// ---- MFMA issue -----------------------------------------------------------------------
// MFMAs are issued from inline asm with the accumulator tied in place ("+v"): SrcC is always
// the destination, so no other value can be allocated into an in-flight MFMA's SrcC
// registers, and the compiler's own MFMA wait-state tables are never relied on.  On gfx950
// those tables were too short for v_mfma_f32_16x16x4_f32 in two ways: the 4th result
// register read through v_accvgpr_read ~8 wait states after the last MFMA came back stale,
// and VALU writes ~11 wait states after an MFMA whose SrcC differed from its destination
// corrupted result elements 2-3.  Rules used here:
//   * each asm block starts with s_nop 1 (VALU-written A/B operand -> MFMA read);
//   * back-to-back MFMAs accumulating in place into the same registers are interlocked by
//     the hardware (measured: 36 clk per dependent 16x16x4 f32 MFMA vs 32 independent);
//   * before any non-MFMA instruction reads an accumulator, drain() holds 24 wait states
//     and takes the accumulator as an operand, so no read can be scheduled above it.
__device__ __forceinline__ void mfma_f32x1(f4& acc, float a, float b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_f32x4(f4& acc, const float4& a, const float4& b) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %1, %5, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %2, %6, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %3, %7, %0\n\t"
      "v_mfma_f32_16x16x4_f32 %0, %4, %8, %0"
      : "+v"(acc)
      : "v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w), "v"(b.x), "v"(b.y), "v"(b.z), "v"(b.w));
}
__device__ __forceinline__ void mfma_bf16x1(f4& acc, const s4& a, const s4& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_bf16x3(f4& acc, const s4& ah, const s4& al, const s4& bh, const s4& bl) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x16_bf16 %0, %1, %3, %0\n\t"
      "v_mfma_f32_16x16x16_bf16 %0, %1, %4, %0\n\t"
      "v_mfma_f32_16x16x16_bf16 %0, %2, %3, %0"
      : "+v"(acc)
      : "v"(ah), "v"(al), "v"(bh), "v"(bl));
}
// gfx950's 32-deep bf16 MFMA: lane l supplies 8 k values of A's row l % 16 and of B's column
// l % 16 (group l / 16); the pairing of A's and B's values is all that matters to the sum.
typedef short s8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ void mfma_bf16x1_k32(f4& acc, const s8& a, const s8& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_bf16x3_k32(f4& acc, const s8& ah, const s8& al, const s8& bh, const s8& bl) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %1, %3, %0\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %1, %4, %0\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %2, %3, %0"
      : "+v"(acc)
      : "v"(ah), "v"(al), "v"(bh), "v"(bl));
}
// The bf16x3 passes with the cross terms in the other order (hi*hi, lo*hi, hi*lo): with the
// operands' roles exchanged this issues the products of mfma_bf16x3(acc, bh, bl, ah, al) in
// that call's order, so the two accumulate bit-identically (one is the other's transpose).
__device__ __forceinline__ void mfma_bf16x3_tr(f4& acc, const s4& ah, const s4& al, const s4& bh, const s4& bl) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x16_bf16 %0, %1, %3, %0\n\t"
      "v_mfma_f32_16x16x16_bf16 %0, %2, %3, %0\n\t"
      "v_mfma_f32_16x16x16_bf16 %0, %1, %4, %0"
      : "+v"(acc)
      : "v"(ah), "v"(al), "v"(bh), "v"(bl));
}
__device__ __forceinline__ void mfma_bf16x3_k32_tr(f4& acc, const s8& ah, const s8& al, const s8& bh, const s8& bl) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %1, %3, %0\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %2, %3, %0\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %1, %4, %0"
      : "+v"(acc)
      : "v"(ah), "v"(al), "v"(bh), "v"(bl));
}
__device__ __forceinline__ void drain(f4& a) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a));
}
__device__ __forceinline__ void drain(f4& a, f4& b) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void drain(f4& a, f4& b, f4& c) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c));
}
__device__ __forceinline__ void drain(f4& a, f4& b, f4& c, f4& d) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}

// ---- one 16x16 output tile: acc += A[0:16, 0:K] * B[0:K, 0:16] ------------------------
// A and B are views already shifted to the tile origin.  K % 16 == 0.  The tile routines
// end with drain(acc): the accumulator is ready for ordinary code when they return.
__device__ __forceinline__ void mma_tile_f32(f4& acc, const View& A, const View& B, int K) {
  const int l = lane_id(), r = l & 15, g = l >> 4;
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += 4) mfma_f32x1(acc, A.at(r, k0 + g), B.at(k0 + g, r));
}

// hi = bf16(x), lo = bf16(x - hi), four packed conversions per float4
__device__ __forceinline__ void split4(const float4& x, s4& hi, s4& lo) {
  const uint32_t h01 = bf16_pack(x.x, x.y), h23 = bf16_pack(x.z, x.w);
  const uint32_t l01 = bf16_pack(x.x - __uint_as_float(h01 << 16), x.y - __uint_as_float(h01 & 0xffff0000u));
  const uint32_t l23 = bf16_pack(x.z - __uint_as_float(h23 << 16), x.w - __uint_as_float(h23 & 0xffff0000u));
  hi = __builtin_bit_cast(s4, make_uint2(h01, h23));
  lo = __builtin_bit_cast(s4, make_uint2(l01, l23));
}
__device__ __forceinline__ s4 round4(const float4& x) {
  return __builtin_bit_cast(s4, make_uint2(bf16_pack(x.x, x.y), bf16_pack(x.z, x.w)));
}

template <bool THREE>
__device__ __forceinline__ void mma_tile_bf16(f4& acc, const View& A, const View& B, int K);

// ---- one 16-wide k block with register operands ----------------------------------------
// k-permuted mapping: within a 16-wide block, lane group g = l/16 owns k = 4g + e, e = 0..3,
// so a lane supplies a = A[l%16][4g .. 4g+3] and b = B[4g .. 4g+3][l%16] as two float4.
// highest: 4 fp32 MFMAs (step e pairs a[e] with b[e]); bf16 modes: one 16x16x16 bf16 MFMA
// whose lane layout is exactly this (bf16x3: hi*hi + hi*lo + lo*hi).
// The 16x16 result layout (lane l holds rows 4g..4g+3 of column l%16) is the B-operand
// layout of the next k block, so a tile produced by one MFMA chain feeds another directly.
// mma16 does not drain: callers chain several and drain() before reading the result.
// The dot mode is a template parameter everywhere an MFMA is issued: a runtime switch would
// put branches between the MFMAs of a chain, and at the merge points the compiler copies
// the accumulator right after the (opaque) asm MFMA -- a read it cannot know to delay.
template <int MODE>
__device__ __forceinline__ void mma16(f4& acc, const float4& a, const float4& b) {
  if constexpr (MODE == DOT_HIGHEST) {
    mfma_f32x4(acc, a, b);
  } else if constexpr (MODE == DOT_BF16X3) {
    s4 ah, al, bh, bl;
    split4(a, ah, al);
    split4(b, bh, bl);
    mfma_bf16x3(acc, ah, al, bh, bl);
  } else {
    mfma_bf16x1(acc, round4(a), round4(b));
  }
}
// Two consecutive 16-wide k blocks at once: (a0, b0) are the lane's operands of block kb,
// (a1, b1) of block kb + 1.  highest: the same 8 fp32 MFMAs as two mma16 calls (identical
// results); the bf16 modes: one 16x16x32 bf16 MFMA per pass on the two blocks' values
// concatenated (lane group g: k = 4 g .. 4 g + 3 of both blocks), half the bf16 issues.
__device__ __forceinline__ s8 cat8(const s4& x, const s4& y) {
  return s8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}
template <int MODE>
__device__ __forceinline__ void mma32(f4& acc, const float4& a0, const float4& b0, const float4& a1, const float4& b1) {
  if constexpr (MODE == DOT_HIGHEST) {
    mfma_f32x4(acc, a0, b0);
    mfma_f32x4(acc, a1, b1);
  } else if constexpr (MODE == DOT_BF16X3) {
    s4 a0h, a0l, a1h, a1l, b0h, b0l, b1h, b1l;
    split4(a0, a0h, a0l);
    split4(a1, a1h, a1l);
    split4(b0, b0h, b0l);
    split4(b1, b1h, b1l);
    mfma_bf16x3_k32(acc, cat8(a0h, a1h), cat8(a0l, a1l), cat8(b0h, b1h), cat8(b0l, b1l));
  } else {
    mfma_bf16x1_k32(acc, cat8(round4(a0), round4(a1)), cat8(round4(b0), round4(b1)));
  }
}
// The transposed product: mma16_tr<MODE>(acc, a, b) takes a as the A operand and b as the B
// operand and issues the products of mma16<MODE>(acc', b, a) in that call's order, so acc ends
// up as the transpose of acc', bit for bit (each MFMA's sum is symmetric in its operands).
// A producer that needs a tile in the other orientation swaps the operands instead of
// transposing the result.
template <int MODE>
__device__ __forceinline__ void mma16_tr(f4& acc, const float4& a, const float4& b) {
  if constexpr (MODE == DOT_BF16X3) {
    s4 ah, al, bh, bl;
    split4(a, ah, al);
    split4(b, bh, bl);
    mfma_bf16x3_tr(acc, ah, al, bh, bl);
  } else {
    mma16<MODE>(acc, a, b);
  }
}
template <int MODE>
__device__ __forceinline__ void mma32_tr(f4& acc, const float4& a0, const float4& b0, const float4& a1, const float4& b1) {
  if constexpr (MODE == DOT_BF16X3) {
    s4 a0h, a0l, a1h, a1l, b0h, b0l, b1h, b1l;
    split4(a0, a0h, a0l);
    split4(a1, a1h, a1l);
    split4(b0, b0h, b0l);
    split4(b1, b1h, b1l);
    mfma_bf16x3_k32_tr(acc, cat8(a0h, a1h), cat8(a0l, a1l), cat8(b0h, b1h), cat8(b0l, b1l));
  } else {
    mma32<MODE>(acc, a0, b0, a1, b1);
  }
}
// acc += sum over the k blocks kb in [k0, K1) of the lane operands a(kb), b(kb): fp32 one block
// at a time (the instruction stream of a plain mma16 loop), the bf16 modes two blocks per
// 32-deep MFMA and a last single block if the count is odd.  k0 must fold to a constant
// (a template value or an unrolled loop index): no branch may sit inside a chain.
template <int MODE, int K1, class FA, class FB>
__device__ __forceinline__ void mma_chain(f4& acc, int k0, FA a, FB b) {
  if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
    for (int kb = k0; kb < K1; ++kb) mma16<MODE>(acc, a(kb), b(kb));
  } else {
#pragma unroll
    for (int kb = k0; kb + 1 < K1; kb += 2) mma32<MODE>(acc, a(kb), b(kb), a(kb + 1), b(kb + 1));
    if ((K1 - k0) & 1) mma16<MODE>(acc, a(K1 - 1), b(K1 - 1));
  }
}
__device__ __forceinline__ float4 f4_to_float4(const f4& x) { return make_float4(x[0], x[1], x[2], x[3]); }

// bf16 tile product for the diagnostics: pairs of 16-wide k blocks on the 32-deep MFMA (the
// operand mapping of mma32), a last single block on the 16-deep one
template <bool THREE>
__device__ __forceinline__ void mma_tile_bf16(f4& acc, const View& A, const View& B, int K) {
  constexpr int MODE = THREE ? DOT_BF16X3 : DOT_DEFAULT;
  const int l = lane_id(), r = l & 15, g = l >> 4;
  auto opa = [&](int k0) {
    const int kk = k0 + 4 * g;
    return make_float4(A.at(r, kk), A.at(r, kk + 1), A.at(r, kk + 2), A.at(r, kk + 3));
  };
  auto opb = [&](int k0) {
    const int kk = k0 + 4 * g;
    return make_float4(B.at(kk, r), B.at(kk + 1, r), B.at(kk + 2, r), B.at(kk + 3, r));
  };
  int k0 = 0;
  for (; k0 + 32 <= K; k0 += 32) mma32<MODE>(acc, opa(k0), opb(k0), opa(k0 + 16), opb(k0 + 16));
  if (k0 < K) mma16<MODE>(acc, opa(k0), opb(k0));
}
__device__ __forceinline__ float4 scale4(const float4& x, float s) { return make_float4(s * x.x, s * x.y, s * x.z, s * x.w); }
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Raw operator inputs are fp32 or bfloat16 (stored as uint16_t bits); the kernels widen them
// to fp32 on load and compute in fp32 from there.
__device__ __forceinline__ float in_val(const float* p) { return *p; }
__device__ __forceinline__ float in_val(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }
__device__ __forceinline__ float4 in_ld4(const float* p) { return ld4(p); }
__device__ __forceinline__ float4 in_ld4(const uint16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                     __uint_as_float(u.y & 0xffff0000u));
}
// Global load with the non-temporal hint, for the last read of a value by any kernel of the
// operator: the line is not kept in the caches, which leaves room for values read again (in
// this kernel, or by a later one).
typedef unsigned u2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ldg4(const float* p) {
  const f4 v = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 in_ldg4(const float* p) { return ldg4(p); }
// LDS DMA (gfx950 global_load_lds_dwordx4): lane i of the wave fetches the 16 bytes at its own
// global address src into LDS at dst + 4 i floats (dst wave-uniform, 16-byte aligned).  No
// registers are involved.  Issued from inline asm, so the compiler does not know of it: it
// neither holds later LDS accesses for it (it cannot tell which LDS it writes) nor counts it in
// its own waits (which then only wait longer: memory operations complete in order).  The
// caller waits for it (s_waitcnt vmcnt(0)) and publishes it with a barrier.  It sets M0, which
// the compiler reserves but does not use in the kernels that call this (no other LDS DMA, GWS
// or message instruction), so the clobber is safe there.
__device__ __forceinline__ void lds_dma16(const float* src, float* dst) {
  const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)dst;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds) : "memory", "m0");
}
// The kernel's argument block (its first and only explicit argument, at offset 0 of the
// kernarg segment) seen through a pointer that is opaque to the optimiser when FRESH: loads
// through it cannot be hoisted out of a loop, so a persistent kernel re-reads (scalar loads)
// each argument where it is used instead of holding them all in SGPRs across the loop.
template <typename A>
__device__ __forceinline__ const __attribute__((address_space(4))) A* kernarg_fresh(bool fresh) {
  auto p = (const __attribute__((address_space(4))) A*)__builtin_amdgcn_kernarg_segment_ptr();
  if (fresh) asm volatile("" : "+s"(p));
  return p;
}
// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding: vmcnt [3:0] and
// [15:14], expcnt [6:4] = 7, lgkmcnt [11:8] = 15)
constexpr int WAIT_VMCNT0 = 0x0F70;
__device__ __forceinline__ float4 in_ldg4(const uint16_t* p) {
  const u2v u = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(p));
  return make_float4(__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xffff0000u), __uint_as_float(u[1] << 16),
                     __uint_as_float(u[1] & 0xffff0000u));
}
__device__ __forceinline__ void st4(float* p, const float4& x) { *reinterpret_cast<float4*>(p) = x; }

// A wave-uniform global address held in SGPRs, opaque to the optimiser: p + (32-bit lane
// offset) then compiles to a scalar-base global load / store (saddr + 32-bit voffset), and
// loop-invariant code motion cannot merge the lane offset into per-block 64-bit sums and keep
// one such VGPR pair live for every block of a loop.  The argument must be wave-uniform.
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) const float cgfloat;
__device__ __forceinline__ cgfloat* sbase(const float* p) {
  cgfloat* q = (cgfloat*)p;
  asm volatile("" : "+s"(q));
  return q;
}
__device__ __forceinline__ gfloat* sbase(float* p) {
  gfloat* q = (gfloat*)p;
  asm volatile("" : "+s"(q));
  return q;
}
__device__ __forceinline__ float4 ld4(cgfloat* p) {
  const f4 v = *reinterpret_cast<const __attribute__((address_space(1))) f4*>(p);
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void stg4(gfloat* p, const float4& x) {
  const f4 v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<__attribute__((address_space(1))) f4*>(p));
}
// Global store with the non-temporal (streaming) hint, for outputs that only a later kernel
// reads: they then do not evict from L2 the inputs that the writing kernel reads again.
__device__ __forceinline__ void stg4(float* p, const float4& x) {
  const f4 v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p));
}
// Plain (cache-allocating) global store, for the WY build's outputs (the scan operands and the
// residual) and the operator's output o.  Measured against the streaming store at config 2: the
// WY build 62.8 -> 59.5 us, and the reverse scan and bwd_pre, which read that residual in the
// backward, 1-3 us faster each (the lines appear to stay in MI355X's 256 MB memory-side cache);
// o, which the caller's loss reads next, -2.5 us per gradient evaluation.  The same switch for
// the backward's intermediates gained nothing, and for its gradients it cost bwd_wy 2-4 us.
__device__ __forceinline__ void stg4_keep(float* p, const float4& x) {
  const f4 v = {x.x, x.y, x.z, x.w};
  *reinterpret_cast<f4*>(p) = v;
}

template <int MODE>
__device__ __forceinline__ void mma_tile(f4& acc, const View& A, const View& B, int K) {
  if constexpr (MODE == DOT_HIGHEST) mma_tile_f32(acc, A, B, K);
  else mma_tile_bf16<MODE == DOT_BF16X3>(acc, A, B, K);
  drain(acc);
}

// mma_tile under a runtime dot mode: the branch encloses whole tiles, each ending in drain(),
// so no accumulator copy can land next to an in-flight MFMA.
__device__ __forceinline__ void mma_tile_rt(int mode, f4& acc, const View& A, const View& B, int K) {
  if (mode == DOT_HIGHEST) mma_tile<DOT_HIGHEST>(acc, A, B, K);
  else if (mode == DOT_BF16X3) mma_tile<DOT_BF16X3>(acc, A, B, K);
  else mma_tile<DOT_DEFAULT>(acc, A, B, K);
}

// Calls f(std::integral_constant<int, mode>) for a runtime dot mode.
template <class F>
inline auto dispatch_mode(int mode, F&& f) {
  if (mode == DOT_HIGHEST) return f(std::integral_constant<int, DOT_HIGHEST>{});
  if (mode == DOT_BF16X3) return f(std::integral_constant<int, DOT_BF16X3>{});
  return f(std::integral_constant<int, DOT_DEFAULT>{});
}

// Scalar dot product of length n under a dot mode (used by the small ladder merges).
// a(i), b(i) are callables.  bf16x3 keeps the three partial sums apart and adds them as
// (hh + hl) + lh, like three separate products summed.
template <class FA, class FB>
__device__ __forceinline__ float dot_mode_scalar(int mode, int lo, int hi, FA a, FB b) {
  if (mode == DOT_HIGHEST) {
    float s = 0.f;
    for (int i = lo; i < hi; ++i) s = fmaf(a(i), b(i), s);
    return s;
  }
  if (mode == DOT_DEFAULT) {
    float s = 0.f;
    for (int i = lo; i < hi; ++i) s = fmaf(bf16_round(a(i)), bf16_round(b(i)), s);
    return s;
  }
  float shh = 0.f, shl = 0.f, slh = 0.f;
  for (int i = lo; i < hi; ++i) {
    const float x = a(i), y = b(i);
    const float xh = bf16_round(x), yh = bf16_round(y);
    const float xl = bf16_round(x - xh), yl = bf16_round(y - yh);
    shh = fmaf(xh, yh, shh);
    shl = fmaf(xh, yl, shl);
    slh = fmaf(xl, yh, slh);
  }
  return (shh + shl) + slh;
}

// Output coordinates of accumulator element r of the calling lane inside a 16x16 tile.
__device__ __forceinline__ int tile_row(int r) { return 4 * (lane_id() >> 4) + r; }
__device__ __forceinline__ int tile_col() { return lane_id() & 15; }

__device__ __forceinline__ float4 add4(const float4& a, const float4& b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 sub4(const float4& a, const float4& b) {
  return make_float4(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w);
}
__device__ __forceinline__ float4 mul4(const float4& a, const float4& b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ float4 san4(const float4& a, float c) {
  return make_float4(sanitize(a.x, c), sanitize(a.y, c), sanitize(a.z, c), sanitize(a.w, c));
}
__device__ __forceinline__ float4 expnp4(const float4& a) {
  return make_float4(exp_nonpos(a.x), exp_nonpos(a.y), exp_nonpos(a.z), exp_nonpos(a.w));
}

// ---- fragment-blocked tiles --------------------------------------------------------------
// An R x C tile in "fragment" layout is stored as 16x16 blocks in row-major block order
// (C/16 blocks per block row); inside a block the float4 of lane l = r + 16 g holds
// M[16 bi + r][16 bj + 4 g .. 4 g + 3].  A wave moves a block with one coalesced 1 KB float4
// access, and lane l's float4 is exactly its operand for one 16-wide k block of mma16 with
// rows = M rows and k = M columns (A operand), or columns = M rows and k = M columns
// (B operand of M^T).  The accumulator of an MFMA tile P (lane l holds P[4 g + e][l % 16])
// is therefore block (bj, bi) of P^T in fragment layout, stored without any shuffle.
__device__ __forceinline__ int frag_blk(int bi, int bj, int C) { return (bi * (C >> 4) + bj) << 8; }
__device__ __forceinline__ int frag_off(int i, int j, int C) {
  return frag_blk(i >> 4, j >> 4, C) + (((i & 15) + ((j & 15) >> 2) * 16) << 2) + (j & 3);
}

// 16x16 tile held in the MFMA result layout (lane l = r + 16 g: column r, rows 4 g .. 4 g + 3)
// -> the same tile in the A-operand layout (lane l: row r, columns 4 g .. 4 g + 3), through a
// per-wave LDS tile with row stride TRP (conflict-free column reads).  Only the issuing wave
// touches `tr`, and LDS operations of one wave complete in order.
constexpr int TRP = 20;
__device__ __forceinline__ float4 wave_transpose16(float* tr, const float4 x, int r, int g) {
  st4(tr + r * TRP + 4 * g, x);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return make_float4(tr[(4 * g) * TRP + r], tr[(4 * g + 1) * TRP + r], tr[(4 * g + 2) * TRP + r],
                     tr[(4 * g + 3) * TRP + r]);
}

// N tiles at once: x[i] (MFMA result / operand layout) -> y[i], the transposed tile, through N
// per-wave LDS tiles of 16 x TRP floats at tr: every write, one wave barrier, every read.
template <int N>
__device__ __forceinline__ void wave_transpose16_n(float* tr, const float4* x, float4* y, int r, int g) {
#pragma unroll
  for (int i = 0; i < N; ++i) st4(tr + i * 16 * TRP + r * TRP + 4 * g, x[i]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float* t = tr + i * 16 * TRP;
    y[i] = make_float4(t[(4 * g) * TRP + r], t[(4 * g + 1) * TRP + r], t[(4 * g + 2) * TRP + r], t[(4 * g + 3) * TRP + r]);
  }
}

// In-chunk cumulative sum of g over the T rows of a (T x D) tile, into LDS sG (ld = LD).
// Thread t owns float4 column t % (D/4) over a run of RUN consecutive rows: it sums its run,
// then adds the totals of the runs above it in order.  Same code in every kernel, so every
// kernel sees bit-identical gc.
// LAST_READ: g is not read again by a later kernel (loaded with the non-temporal hint).
template <int D, int LD, int NTHREADS, bool LAST_READ = false, typename TIn>
__device__ __forceinline__ void chunk_cumsum(const TIn* __restrict__ g, float* sG) {
  constexpr int NQ = D / 4, NSEG = NTHREADS / NQ, RUN = T / NSEG;
  static_assert(NTHREADS % NQ == 0 && T % NSEG == 0 && RUN >= 1, "cumsum split");
  const int t = threadIdx.x, d = 4 * (t % NQ), s = t / NQ;
  float4 x[RUN];
#pragma unroll
  for (int i = 0; i < RUN; ++i) x[i] = LAST_READ ? in_ldg4(g + (s * RUN + i) * D + d) : in_ld4(g + (s * RUN + i) * D + d);
#pragma unroll
  for (int i = 1; i < RUN; ++i) x[i] = add4(x[i - 1], x[i]);
  st4(sG + (s * RUN + RUN - 1) * LD + d, x[RUN - 1]);
  __syncthreads();
  // the run totals above are read all at once, then added in order
  float4 tot[NSEG - 1];
#pragma unroll
  for (int s2 = 0; s2 < NSEG - 1; ++s2) tot[s2] = ld4(sG + (s2 * RUN + RUN - 1) * LD + d);
  float4 off = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int s2 = 0; s2 < NSEG - 1; ++s2) off = s2 < s ? add4(off, tot[s2]) : off;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < RUN; ++i) st4(sG + (s * RUN + i) * LD + d, add4(off, x[i]));
  __syncthreads();
}

// chunk_cumsum<D, ., NVIRT> for the columns [c0, c0 + 4 NQP) only, run by NREAL threads, with the
// result in fragment layout (T x 4 NQP).  Every virtual thread (s, cq) of chunk_cumsum that owns
// one of those columns (float4 column cq, rows s RUN .. s RUN + RUN - 1) is run by one real thread
// (the first NSEG NQP threads, several virtual threads each if there are fewer real ones), adding
// in exactly its order, so gc is bit-identical to chunk_cumsum's.  load() issues the g loads
// (into registers); run() needs NSEG x NQP float4 of LDS for the run totals, is called by every
// thread and ends with a barrier.
template <int D, int NVIRT, int NREAL, int NQP>
struct CumsumPass {
  static constexpr int NQ = D / 4, NSEG = NVIRT / NQ, RUN = T / NSEG, NACT = NSEG * NQP;
  static constexpr int NV = (NACT + NREAL - 1) / NREAL;
  static_assert(NVIRT % NQ == 0 && T % NSEG == 0 && (NACT <= NREAL || NACT % NREAL == 0), "cumsum split");
  float4 x[NV][RUN];
  __device__ __forceinline__ bool active(int m) const { return NACT >= NREAL || (int)threadIdx.x < NACT; }
  __device__ __forceinline__ int seg(int m) const { return (threadIdx.x + NREAL * m) / NQP; }
  __device__ __forceinline__ int col(int m) const { return (threadIdx.x + NREAL * m) % NQP; }
  template <typename TIn>
  __device__ __forceinline__ void load(const TIn* __restrict__ g, int c0) {
#pragma unroll
    for (int m = 0; m < NV; ++m)
      if (active(m)) {
#pragma unroll
        for (int i = 0; i < RUN; ++i) x[m][i] = in_ld4(g + (seg(m) * RUN + i) * D + c0 + 4 * col(m));
      }
  }
  // the loaded rows are gc already (the caller's in-chunk cumsum): store them as they are
  __device__ __forceinline__ void store_as_is(float* sGf) {
#pragma unroll
    for (int m = 0; m < NV; ++m)
      if (active(m)) {
#pragma unroll
        for (int i = 0; i < RUN; ++i) st4(sGf + frag_off(seg(m) * RUN + i, 4 * col(m), 4 * NQP), x[m][i]);
      }
    __syncthreads();
  }
  __device__ __forceinline__ void run(float* sGf, float4* sTot) {
#pragma unroll
    for (int m = 0; m < NV; ++m)
      if (active(m)) {
#pragma unroll
        for (int i = 1; i < RUN; ++i) x[m][i] = add4(x[m][i - 1], x[m][i]);
        sTot[seg(m) * NQP + col(m)] = x[m][RUN - 1];
      }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NV; ++m)
      if (active(m)) {
        const int s = seg(m), cq = col(m);
        float4 off = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s2 = 0; s2 < s; ++s2) off = add4(off, sTot[s2 * NQP + cq]);
#pragma unroll
        for (int i = 0; i < RUN; ++i) st4(sGf + frag_off(s * RUN + i, 4 * cq, 4 * NQP), add4(off, x[m][i]));
      }
    __syncthreads();
  }
};

}  // namespace gdn2
