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

namespace gdn2 {

constexpr int T = 64;        // chunk length (cfg.bt) supported by the kernels
constexpr int WAVE = 64;

enum DotMode : int { DOT_HIGHEST = 0, DOT_BF16X3 = 1, DOT_DEFAULT = 2 };
enum DiagMode : int { DIAG_BTL = 0, DIAG_LEAN = 1 };

typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / WAVE; }

__device__ __forceinline__ float sanitize(float x, float c) {
  if (x != x) return 0.f;
  return fminf(fmaxf(x, -c), c);
}

__device__ __forceinline__ float exp_nonpos(float x) { return expf(fminf(x, 0.f)); }

// ---- bfloat16 helpers: round-to-nearest-even, NaN kept quiet ------------------------
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
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

// ---- one 16x16 output tile: acc += A[0:16, 0:K] * B[0:K, 0:16] ------------------------
// A and B are views already shifted to the tile origin.  K % 16 == 0.
__device__ __forceinline__ void mma_tile_f32(f4& acc, const View& A, const View& B, int K) {
  const int l = lane_id(), r = l & 15, g = l >> 4;
#pragma unroll 4
  for (int k0 = 0; k0 < K; k0 += 4)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A.at(r, k0 + g), B.at(k0 + g, r), acc, 0, 0, 0);
}

template <bool THREE>
__device__ __forceinline__ void mma_tile_bf16(f4& acc, const View& A, const View& B, int K) {
  const int l = lane_id(), r = l & 15, g = l >> 4;
  for (int k0 = 0; k0 < K; k0 += 16) {
    s4 ah, bh, al, bl;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = A.at(r, k0 + 4 * g + e);
      const float b = B.at(k0 + 4 * g + e, r);
      const uint32_t ha = bf16_bits(a), hb = bf16_bits(b);
      ah[e] = (short)ha;
      bh[e] = (short)hb;
      if (THREE) {
        al[e] = (short)bf16_bits(a - bf16_val(ha));
        bl[e] = (short)bf16_bits(b - bf16_val(hb));
      }
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, acc, 0, 0, 0);
    if (THREE) {
      acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bl, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bh, acc, 0, 0, 0);
    }
  }
}

__device__ __forceinline__ void mma_tile(int mode, f4& acc, const View& A, const View& B, int K) {
  if (mode == DOT_HIGHEST) mma_tile_f32(acc, A, B, K);
  else if (mode == DOT_BF16X3) mma_tile_bf16<true>(acc, A, B, K);
  else mma_tile_bf16<false>(acc, A, B, K);
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

// In-chunk cumulative sum of g over the T rows of a (T x D) tile, into LDS sG (ld = LD).
// Column d is owned by NSEG threads, each summing a contiguous run of rows, followed by an
// offset pass.  Same code in every kernel, so every kernel sees bit-identical gc.
template <int D, int LD, int NTHREADS>
__device__ __forceinline__ void chunk_cumsum(const float* __restrict__ g, float* sG) {
  constexpr int NSEG = NTHREADS / D;          // segments per column
  constexpr int RUN = T / NSEG;               // rows per segment
  static_assert(NTHREADS % D == 0 && T % NSEG == 0, "cumsum split");
  const int t = threadIdx.x, d = t % D, s = t / D;
  float acc = 0.f;
#pragma unroll 4
  for (int i = 0; i < RUN; ++i) {
    const int row = s * RUN + i;
    acc += g[row * D + d];
    sG[row * LD + d] = acc;
  }
  __syncthreads();
  // offset pass: segment s adds the totals of segments 0..s-1 (sequential order)
  float off = 0.f;
  for (int s2 = 0; s2 < s; ++s2) off += sG[(s2 * RUN + RUN - 1) * LD + d];
  __syncthreads();
  if (s > 0) {
    for (int i = 0; i < RUN; ++i) {
      const int row = s * RUN + i;
      sG[row * LD + d] += off;
    }
  }
  __syncthreads();
}

}  // namespace gdn2
