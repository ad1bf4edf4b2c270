// Forward kernels of the GDN-2 operator on gfx950.
//
//   wy_fwd_kernel   one workgroup per chunk (B*H*nc of them): in-chunk cumulative decay gc,
//                   gated scores Aqk / Akk (two-level block-local rescaling, BTL or lean
//                   diagonal), unit-lower-triangular inverse A = (I + (1-eps) Akk)^-1 by leaf
//                   forward substitution + block doubling in LDS, then Wp = A (b*k*e^gc) and
//                   U = A (w*v) on MFMA, plus the gated Kg, Qg and gamma = gc[T-1].
//                   Semantics: fwd/scores.py:42-87, fwd/solve.py:9-48, fwd/cd_slim.py:14-21.
//   (the forward state scan is in gdn2_scan.hip)
#include "gdn2_kernels.hpp"

namespace gdn2 {

// ------------------------------------------------------------------------------------
// WY build
// ------------------------------------------------------------------------------------
template <int D>
struct WyFwdLayout {
  static constexpr int LD = D + 4, LT = T + 4;
  static constexpr int R0 = T * LD;          // gc, later w*v
  static constexpr int R1 = 3 * 32 * LD;     // piece staging, later b*k*e^gc, merge temp
  static constexpr int OFF_G = 0, OFF_ST = R0, OFF_S = R0 + R1;
  static constexpr int OFF_K = OFF_S + T * LT, OFF_I = OFF_K + T * LT;
  static constexpr int TOTAL = OFF_I + T * LT;
  static_assert(R1 >= T * LD && R1 >= T * LT, "staging region too small");
};

template <int D, int DOT>
__global__ __launch_bounds__(512) void wy_fwd_kernel(WyFwdArgs a) {
  using Lay = WyFwdLayout<D>;
  constexpr int LD = Lay::LD, LT = Lay::LT, NT = 512, NW = NT / WAVE;
  __shared__ float smem[Lay::TOTAL];
  float* sG = smem + Lay::OFF_G;
  float* sSt = smem + Lay::OFF_ST;
  float* sS = smem + Lay::OFF_S;
  float* sK = smem + Lay::OFF_K;
  float* sI = smem + Lay::OFF_I;
  const Cfg& cf = a.cfg;
  const float clip = cf.clip;
  const int chunk = blockIdx.x;
  const size_t tb = (size_t)chunk * T * D;
  const size_t sb = (size_t)chunk * T * T;
  const float* __restrict__ q = a.q + tb;
  const float* __restrict__ k = a.k + tb;
  const float* __restrict__ b = a.b + tb;
  const float* __restrict__ w = a.w + tb;
  const float* __restrict__ v = a.v + tb;
  const int tid = threadIdx.x, wv = wave_id();

  // 1. gc = cumsum(g) inside the chunk
  chunk_cumsum<D, LD, NT>(a.g + tb, sG);

  // 2. gated k / q and gamma (cd_slim.py:17-21): kg = san(k e^{min(gl-gc,0)}), qg = san(q e^{min(gc,0)});
  //    each thread does 4 consecutive rows of one column (row-major and transposed stores)
  for (int e = tid; e < (T / 4) * D; e += NT) {
    const int d = e % D, i0 = 4 * (e / D);
    const float gl = sG[(T - 1) * LD + d];
    float kv[4], qv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + r;
      const float gi = sG[i * LD + d];
      kv[r] = sanitize(k[i * D + d] * exp_nonpos(gl - gi), clip);
      qv[r] = sanitize(q[i * D + d] * exp_nonpos(gi), clip);
      if (a.kg) a.kg[tb + i * D + d] = kv[r];
      if (a.qg) a.qg[tb + i * D + d] = qv[r];
    }
    if (a.kgT) st4(a.kgT + tb + (size_t)d * T + i0, make_float4(kv[0], kv[1], kv[2], kv[3]));
    if (a.qgT) st4(a.qgT + tb + (size_t)d * T + i0, make_float4(qv[0], qv[1], qv[2], qv[3]));
  }
  if (tid < D) a.gl[(size_t)chunk * D + tid] = sG[(T - 1) * LD + tid];

  // 3. scores, piece by piece (scores.py:42-75)
  for (int pi = 0; pi < cf.pieces.n; ++pi) {
    const Piece pc = cf.pieces.p[pi];
    const int P = pc.P;
    const bool lean = (pc.kind == 1 && cf.diag == DIAG_LEAN);
    float* sQs = sSt;
    float* sBs = sSt + 32 * LD;
    float* sKs = sSt + 64 * LD;
    for (int e = tid; e < P * D; e += NT) {
      const int i = e / D, d = e % D;
      const int row = pc.row0 + i, col = pc.col0 + i;
      const float ra = lean ? 1.f : piece_row_leg(pc, sG, LD, row, d);
      const float cb = lean ? 1.f : piece_col_leg(pc, sG, LD, col, d);
      sQs[i * LD + d] = q[row * D + d] * ra;
      sBs[i * LD + d] = (b[row * D + d] * k[row * D + d]) * ra;
      sKs[i * LD + d] = k[col * D + d] * cb;
    }
    __syncthreads();
    if (!lean) {
      const int nt1 = P / 16, ntm = nt1 * nt1;
      for (int t = wv; t < 2 * ntm; t += NW) {
        const int mat = t / ntm, ti = (t % ntm) / nt1, tj = t % nt1;
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        mma_tile<DOT>(acc, rm(mat == 0 ? sQs : sBs, LD).shift(ti * 16, 0),
                 tr(sKs, LD).shift(0, tj * 16), D);
        float* out = mat == 0 ? sS : sK;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = pc.row0 + ti * 16 + tile_row(r), j = pc.col0 + tj * 16 + tile_col();
          out[i * LT + j] = mat == 0 ? cf.scale * acc[r] : acc[r];
        }
      }
    } else {
      // lean diagonal (scores.py:34-39): exact exp(clip(gc_i - gc_j, +-diff_clip)) per element
      const float dc = cf.diff_clip;
      for (int e = tid; e < P * P; e += NT) {
        const int i = e / P, j = e % P;
        const int row = pc.row0 + i, col = pc.col0 + j;
        float sq = 0.f, sk = 0.f;
        for (int d = 0; d < D; ++d) {
          const float E = expf(fminf(fmaxf(sG[row * LD + d] - sG[col * LD + d], -dc), dc));
          const float kj = sKs[j * LD + d];
          sq += (sQs[i * LD + d] * E) * kj;
          sk += (sBs[i * LD + d] * E) * kj;
        }
        sS[row * LT + col] = cf.scale * sq;
        sK[row * LT + col] = sk;
      }
    }
    __syncthreads();
  }

  // 4. masks + sanitize (scores.py:84-87); Se = (1-eps) Akk for the solve (solve.py:25)
  for (int e = tid; e < T * (T / 4); e += NT) {
    const int j = e % T, i0 = 4 * (e / T);
    float av[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + r;
      const float aq = j <= i ? sanitize(sS[i * LT + j], clip) : 0.f;
      const float ak = j < i ? sanitize(sK[i * LT + j], clip) : 0.f;
      av[r] = aq;
      sS[i * LT + j] = aq;
      if (a.aqk) a.aqk[sb + i * T + j] = aq;
      if (a.akk) a.akk[sb + i * T + j] = ak;
      sK[i * LT + j] = ak * cf.ome;
      sI[i * LT + j] = 0.f;
    }
    if (a.aqkT) st4(a.aqkT + sb + (size_t)j * T + i0, make_float4(av[0], av[1], av[2], av[3]));
  }
  __syncthreads();

  // 5. inverse of (I + Se): leaves by forward substitution (solve.py:9-18) ...
  const int mb = cf.mb;
  if (tid < T) {
    const int base = (tid / mb) * mb, c = tid % mb;
    for (int i = 0; i < mb; ++i) {
      float s = 0.f;
      for (int j = 0; j < i; ++j) s = fmaf(sK[(base + i) * LT + base + j], sI[(base + j) * LT + base + c], s);
      sI[(base + i) * LT + base + c] = (i == c ? 1.f : 0.f) - s;
    }
  }
  __syncthreads();
  // ... then block doubling X <- [[top, 0], [-bot (S_l top), bot]] (solve.py:30-43)
  float* sM = sSt;
  for (int bb = mb; bb < T; bb *= 2) {
    const int nm = T / (2 * bb), per = bb * bb;
    for (int e = tid; e < nm * per; e += NT) {
      const int m = e / per, i = (e % per) / bb, j = e % bb, i0 = m * 2 * bb;
      const float* srow = sK + (i0 + bb + i) * LT + i0;
      const float* tcol = sI + i0 * LT + i0 + j;
      sM[(i0 + bb + i) * LT + i0 + j] = dot_mode_scalar(
          cf.solve_mode, j, bb, [&](int kk) { return srow[kk]; }, [&](int kk) { return tcol[kk * LT]; });
    }
    __syncthreads();
    for (int e = tid; e < nm * per; e += NT) {
      const int m = e / per, i = (e % per) / bb, j = e % bb, i0 = m * 2 * bb;
      const float* brow = sI + (i0 + bb + i) * LT + i0 + bb;
      const float* mcol = sM + (i0 + bb) * LT + i0 + j;
      sI[(i0 + bb + i) * LT + i0 + j] = -dot_mode_scalar(
          cf.solve_mode, 0, i + 1, [&](int kk) { return brow[kk]; }, [&](int kk) { return mcol[kk * LT]; });
    }
    __syncthreads();
  }
  for (int e = tid; e < T * T; e += NT) {
    const int i = e / T, j = e % T;
    const float x = sanitize(sI[i * LT + j], clip);
    sI[i * LT + j] = x;
    if (a.A) a.A[sb + e] = x;
  }
  __syncthreads();

  // 6. WY operands: b*k*e^{min(gc,0)} and w*v (cd_slim.py:17-18)
  float* sX = sSt;
  float* sY = sG;
  for (int e = tid; e < T * D; e += NT) {
    const int i = e / D, d = e % D;
    sX[i * LD + d] = (b[e] * k[e]) * exp_nonpos(sG[i * LD + d]);
  }
  __syncthreads();
  for (int e = tid; e < T * D; e += NT) {
    const int i = e / D, d = e % D;
    sY[i * LD + d] = w[e] * v[e];
  }
  __syncthreads();

  // 7. Wp = san(A kb), U = san(A wv); A is unit lower triangular so row tile ti only needs
  //    the first (ti+1)*16 columns of A.
  {
    constexpr int NTJ = D / 16, NTM = (T / 16) * NTJ;
    for (int t = wv; t < 2 * NTM; t += NW) {
      const int mat = t / NTM, ti = (t % NTM) / NTJ, tj = t % NTJ;
      f4 acc = {0.f, 0.f, 0.f, 0.f};
      mma_tile<DOT>(acc, rm(sI, LT).shift(ti * 16, 0), rm(mat ? sY : sX, LD).shift(0, tj * 16),
               (ti + 1) * 16);
      float* out = mat ? a.u : a.wp;
      float* outT = mat ? a.uT : a.wpT;
      const float4 x = make_float4(sanitize(acc[0], clip), sanitize(acc[1], clip), sanitize(acc[2], clip),
                                   sanitize(acc[3], clip));
      const int i0 = ti * 16 + tile_row(0), d = tj * 16 + tile_col();
      if (out) {
        out[tb + (i0 + 0) * D + d] = x.x;
        out[tb + (i0 + 1) * D + d] = x.y;
        out[tb + (i0 + 2) * D + d] = x.z;
        out[tb + (i0 + 3) * D + d] = x.w;
      }
      if (outT) st4(outT + tb + (size_t)d * T + i0, x);     // the 4 rows of a lane are consecutive
    }
  }
}

// ------------------------------------------------------------------------------------
// diagnostics: plain GEMM through the MFMA tile routine
// ------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256) void gemm_probe_kernel(const float* A, const float* B, float* C, int M, int N,
                                                         int K) {
  __shared__ float sA[64 * 132];
  __shared__ float sB[128 * 68];
  const int tid = threadIdx.x;
  for (int e = tid; e < M * K; e += 256) sA[(e / K) * 132 + e % K] = A[e];
  for (int e = tid; e < K * N; e += 256) sB[(e / N) * 68 + e % N] = B[e];
  __syncthreads();
  const int nti = M / 16, ntj = N / 16;
  for (int t = wave_id(); t < nti * ntj; t += 4) {
    const int ti = t / ntj, tj = t % ntj;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    mma_tile<MODE>(acc, rm(sA, 132).shift(ti * 16, 0), rm(sB, 68).shift(0, tj * 16), K);
#pragma unroll
    for (int r = 0; r < 4; ++r) C[(ti * 16 + tile_row(r)) * N + tj * 16 + tile_col()] = acc[r];
  }
}

hipError_t launch_gemm_probe(int mode, const float* A, const float* B, float* C, int M, int N, int K,
                             hipStream_t s) {
  dispatch_mode(mode, [&](auto m) {
    hipLaunchKernelGGL(gemm_probe_kernel<decltype(m)::value>, dim3(1), dim3(256), 0, s, A, B, C, M, N, K);
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_wy_fwd(int D, const WyFwdArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.dot_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((wy_fwd_kernel<128, M>), dim3(a.n_chunks), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((wy_fwd_kernel<64, M>), dim3(a.n_chunks), dim3(512), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

}  // namespace gdn2
