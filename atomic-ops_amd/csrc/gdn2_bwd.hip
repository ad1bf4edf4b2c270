// Backward kernels of the GDN-2 operator on gfx950 (the reference fuses all of this into
// one reverse loop per (batch, head), bwd/mega.py:9-58; here the sequential part and the
// chunk-parallel part are separate launches so that the chunk-parallel part fills the GPU).
//
//   (the reverse state scan, dv_new and dh_next per chunk, is in gdn2_scan.hip)
//   bwd_state_kernel one workgroup per chunk: the reductions over the value dimension
//                      dQg = (s dO) h_pre^T, dWp = -dv_new h_pre^T, dKg = v_new dh_next^T
//                    and the row sums sum_v dh_next * h_pre                 (mega.py:38-40,50)
//   bwd_wy_kernel    one workgroup per chunk: dAqk, dA, dkb, dwv, the WY-inverse backward
//                    dAkk = -(1-eps) strict(A^T (dA A^T)), the elementwise gate gradients,
//                    B4 (VJP of the two-level scores) and B5 (reverse cumsum)
//                                                     (mega.py:32-59, bwd/b4.py:45-97)
#include "gdn2_kernels.hpp"

namespace gdn2 {

template <int LD>
__device__ __forceinline__ void load_rows(float* dst, const float* __restrict__ src, int rows, int cols,
                                          int tid, int nt) {
  const float4* s4p = reinterpret_cast<const float4*>(src);
  for (int e = tid; e < rows * cols / 4; e += nt) {
    const int i = (4 * e) / cols, d = (4 * e) % cols;
    *reinterpret_cast<float4*>(dst + i * LD + d) = s4p[e];
  }
}

// ------------------------------------------------------------------------------------
template <int D>
struct StateLayout {
  static constexpr int LD = D + 4, RB = 32;
  static constexpr int OFF_DO = 0, OFF_DV = T * LD, OFF_VN = 2 * T * LD;
  static constexpr int OFF_HP = 3 * T * LD, OFF_DH = OFF_HP + RB * LD;
  static constexpr int TOTAL = OFF_DH + RB * LD;
};

template <int D, int B3>
__global__ __launch_bounds__(512) void bwd_state_kernel(BwdStateArgs a) {
  using Lay = StateLayout<D>;
  constexpr int LD = Lay::LD, RB = Lay::RB, NT = 512, NW = 8;
  __shared__ float smem[Lay::TOTAL];
  float* sdO = smem + Lay::OFF_DO;
  float* sDV = smem + Lay::OFF_DV;
  float* sVn = smem + Lay::OFF_VN;
  float* sHp = smem + Lay::OFF_HP;
  float* sDH = smem + Lay::OFF_DH;
  const Cfg& cf = a.cfg;
  const int chunk = blockIdx.x, tid = threadIdx.x, wv = wave_id();
  const size_t tb = (size_t)chunk * T * D, hb = (size_t)chunk * D * D;
  load_rows<LD>(sdO, a.dout + tb, T, D, tid, NT);
  load_fragT<LD>(sDV, a.dv_new_f + tb, D, T, 0, T, tid, NT);
  load_fragT<LD>(sVn, a.v_new_f + tb, D, T, 0, T, tid, NT);
  for (int rb = 0; rb < D / RB; ++rb) {
    if (rb) __syncthreads();
    load_fragT<LD>(sHp, a.h_pre_f + hb, D, D, rb * RB, RB, tid, NT);
    load_fragT<LD>(sDH, a.dh_next_f + hb, D, D, rb * RB, RB, tid, NT);
    __syncthreads();
    // 3 outputs x 4 row tiles x 2 column tiles (this block of RB key rows)
    for (int t = wv; t < 24; t += NW) {
      const int mat = t / 8, ti = (t % 8) / 2, tj = t % 2;
      f4 acc = {0.f, 0.f, 0.f, 0.f};
      const View A = mat == 0 ? rm(sdO, LD, cf.scale) : (mat == 1 ? rm(sDV, LD, -1.f) : rm(sVn, LD));
      const View B = tr(mat == 2 ? sDH : sHp, LD);
      mma_tile<B3>(acc, A.shift(ti * 16, 0), B.shift(0, tj * 16), D);
      float* out = mat == 0 ? a.dqg : (mat == 1 ? a.dwp : a.dkg);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = ti * 16 + tile_row(r), d = rb * RB + tj * 16 + tile_col();
        out[tb + i * D + d] = acc[r];
      }
    }
    // sum_v dh_next * h_pre for the RB key rows: 16 threads per row, then a fixed-order combine
    {
      const int row = tid / 16, part = tid % 16;
      float s = 0.f;
      for (int v = part; v < D; v += 16) s = fmaf(sDH[row * LD + v], sHp[row * LD + v], s);
      s += __shfl_xor(s, 8, 16);
      s += __shfl_xor(s, 4, 16);
      s += __shfl_xor(s, 2, 16);
      s += __shfl_xor(s, 1, 16);
      if (part == 0) a.dlast[(size_t)chunk * D + rb * RB + row] = s;
    }
  }
}

// ------------------------------------------------------------------------------------
template <int D>
struct BwdWyLayout {
  static constexpr int LD = D + 4, LT = T + 4;
  static constexpr int OFF_G = 0, OFF_X = T * LD, OFF_Y = 2 * T * LD;
  static constexpr int OFF_DAQ = 3 * T * LD, OFF_DA = OFF_DAQ + T * LT, OFF_A = OFF_DA + T * LT;
  static constexpr int OFF_COL = OFF_A + T * LT;
  static constexpr int TOTAL = OFF_COL + D;
  static_assert(2 * T * LD >= 3 * 32 * LD, "B4 staging must fit in X+Y");
};

// Tiles of a T x D output owned by wave w: column strip w % (D/16); row tiles
// w / (D/16) + m * (8 / (D/16)), m = 0..NTW-1.
template <int D>
struct Strip {
  static constexpr int NS = D / 16, NTW = (T / 16) * NS / 8, STEP = 8 / NS;
  __device__ static int strip(int w) { return w % NS; }
  __device__ static int rtile(int w, int m) { return w / NS + m * STEP; }
};

template <int D, int B3>
__global__ __launch_bounds__(512) void bwd_wy_kernel(BwdWyArgs a) {
  using Lay = BwdWyLayout<D>;
  using St = Strip<D>;
  constexpr int LD = Lay::LD, LT = Lay::LT, NT = 512, NW = 8, NTW = St::NTW;
  __shared__ float smem[Lay::TOTAL];
  float* sG = smem + Lay::OFF_G;
  float* sX = smem + Lay::OFF_X;
  float* sY = smem + Lay::OFF_Y;
  float* sDAq = smem + Lay::OFF_DAQ;
  float* sDA = smem + Lay::OFF_DA;
  float* sA = smem + Lay::OFF_A;
  float* sCol = smem + Lay::OFF_COL;
  const Cfg& cf = a.cfg;
  const float clip = cf.clip, scale = cf.scale;
  const int chunk = blockIdx.x, tid = threadIdx.x, wv = wave_id();
  const size_t tb = (size_t)chunk * T * D, sb = (size_t)chunk * T * T;
  const float* __restrict__ q = a.q + tb;
  const float* __restrict__ k = a.k + tb;
  const float* __restrict__ b = a.b + tb;
  const float* __restrict__ w = a.w + tb;
  const float* __restrict__ v = a.v + tb;
  const int strip = St::strip(wv);
  const int dcol = strip * 16 + tile_col();

  chunk_cumsum<D, LD, NT>(a.g + tb, sG);

  // dAqk = (dO v_new^T) * causal                                     (mega.py:32)
  load_rows<LD>(sX, a.dout + tb, T, D, tid, NT);
  load_fragT<LD>(sY, a.v_new_f + tb, D, T, 0, T, tid, NT);
  load_rows<LT>(sA, a.A + sb, T, T, tid, NT);
  __syncthreads();
  for (int t = wv; t < 16; t += NW) {
    const int ti = t / 4, tj = t % 4;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    mma_tile<B3>(acc, rm(sX, LD).shift(ti * 16, 0), tr(sY, LD).shift(0, tj * 16), D);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = ti * 16 + tile_row(r), j = tj * 16 + tile_col();
      sDAq[i * LT + j] = j <= i ? acc[r] : 0.f;
    }
  }
  __syncthreads();

  // dA = san(dWp kb^T + dv_new (w v)^T)                               (mega.py:41)
  f4 accA[2];
  accA[0] = f4{0.f, 0.f, 0.f, 0.f};
  accA[1] = f4{0.f, 0.f, 0.f, 0.f};
  load_rows<LD>(sX, a.dwp + tb, T, D, tid, NT);
  for (int e = tid; e < T * D; e += NT) {
    const int i = e / D, d = e % D;
    sY[i * LD + d] = (b[e] * k[e]) * exp_nonpos(sG[i * LD + d]);
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int t = wv + 8 * m, ti = t / 4, tj = t % 4;
    mma_tile<B3>(accA[m], rm(sX, LD).shift(ti * 16, 0), tr(sY, LD).shift(0, tj * 16), D);
  }
  __syncthreads();
  load_fragT<LD>(sX, a.dv_new_f + tb, D, T, 0, T, tid, NT);
  for (int e = tid; e < T * D; e += NT) {
    const int i = e / D, d = e % D;
    sY[i * LD + d] = w[e] * v[e];
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int t = wv + 8 * m, ti = t / 4, tj = t % 4;
    f4 acc2 = {0.f, 0.f, 0.f, 0.f};
    mma_tile<B3>(acc2, rm(sX, LD).shift(ti * 16, 0), tr(sY, LD).shift(0, tj * 16), D);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = ti * 16 + tile_row(r), j = tj * 16 + tile_col();
      sDA[i * LT + j] = sanitize(accA[m][r] + acc2[r], clip);
    }
  }
  __syncthreads();

  // tmp = san(dA A^T) into X; dAkk = san(-(1-eps) A^T tmp * strict) into sDA  (mega.py:43-44)
  float* sTmp = sX;
  for (int t = wv; t < 16; t += NW) {
    const int ti = t / 4, tj = t % 4;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    mma_tile<B3>(acc, rm(sDA, LT).shift(ti * 16, 0), tr(sA, LT).shift(0, tj * 16), T);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = ti * 16 + tile_row(r), j = tj * 16 + tile_col();
      sTmp[i * LT + j] = sanitize(acc[r], clip);
    }
  }
  __syncthreads();
  {
    f4 accK[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int t = wv + 8 * m, ti = t / 4, tj = t % 4;
      accK[m] = f4{0.f, 0.f, 0.f, 0.f};
      mma_tile<B3>(accK[m], tr(sA, LT).shift(ti * 16, 0), rm(sTmp, LT).shift(0, tj * 16), T);
    }
    __syncthreads();   // all reads of sDA (tmp GEMM) and sTmp done before overwriting
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int t = wv + 8 * m, ti = t / 4, tj = t % 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = ti * 16 + tile_row(r), j = tj * 16 + tile_col();
        sDA[i * LT + j] = j < i ? sanitize(-accK[m][r] * cf.ome, clip) : 0.f;
      }
    }
  }
  // last-row decay gradient (mega.py:50): sum_i dkg*kg*mkg + e^gamma * sum_v(dh_next*h_pre) * mdec
  if (tid < D) {
    const int d = tid;
    const float gl = sG[(T - 1) * LD + d];
    float s = 0.f;
    for (int i = 0; i < T; ++i) {
      const float gi = sG[i * LD + d];
      const float kg = sanitize(k[i * D + d] * exp_nonpos(gl - gi), clip);
      const float mkg = (gl - gi) < 0.f ? 1.f : 0.f;
      s += (a.dkg[tb + i * D + d] * kg) * mkg;
    }
    const float dec = exp_nonpos(gl), mdec = gl < 0.f ? 1.f : 0.f;
    sCol[d] = s + dec * a.dlast[(size_t)chunk * D + d] * mdec;
  }

  // B4: VJP of the two-level scores, piece by piece (bwd/b4.py:45-97)
  f4 bq[NTW], bbk[NTW], bk[NTW], bgc[NTW];
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    bq[m] = f4{0.f, 0.f, 0.f, 0.f};
    bbk[m] = bq[m];
    bk[m] = bq[m];
    bgc[m] = bq[m];
  }
  float* sQt = sX;
  float* sBt = sX + 32 * LD;
  float* sKt = sX + 64 * LD;
  for (int pi = 0; pi < cf.pieces.n; ++pi) {
    const Piece pc = cf.pieces.p[pi];
    const int P = pc.P;
    const bool lean = (pc.kind == 1 && cf.diag == DIAG_LEAN);
    __syncthreads();
    for (int e = tid; e < P * D; e += NT) {
      const int i = e / D, d = e % D;
      const int row = pc.row0 + i, col = pc.col0 + i;
      const float ra = lean ? 1.f : piece_row_leg(pc, sG, LD, row, d);
      const float cb = lean ? 1.f : piece_col_leg(pc, sG, LD, col, d);
      sQt[i * LD + d] = q[row * D + d] * ra;
      sBt[i * LD + d] = (b[row * D + d] * k[row * D + d]) * ra;
      sKt[i * LD + d] = k[col * D + d] * cb;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NTW; ++m) {
      const int rt = St::rtile(wv, m);
      const int r0 = 16 * rt;
      if (!lean) {
        if (r0 >= pc.row0 && r0 < pc.row0 + P) {     // rows of the piece: dq, dbk
          const int lr = r0 - pc.row0;
          f4 dqt = {0.f, 0.f, 0.f, 0.f}, dbt = {0.f, 0.f, 0.f, 0.f};
          mma_tile<DOT_HIGHEST>(dqt, rm(sDAq, LT).shift(r0, pc.col0), rm(sKt, LD).shift(0, strip * 16), P);
          mma_tile<DOT_HIGHEST>(dbt, rm(sDA, LT).shift(r0, pc.col0), rm(sKt, LD).shift(0, strip * 16), P);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = r0 + tile_row(r), il = lr + tile_row(r), d = dcol;
            const float ra = piece_row_leg(pc, sG, LD, i, d);
            const float x = scale * dqt[r];
            bq[m][r] += x * ra;
            bbk[m][r] += dbt[r] * ra;
            bgc[m][r] += x * sQt[il * LD + d] + dbt[r] * sBt[il * LD + d];
          }
        }
        if (r0 >= pc.col0 && r0 < pc.col0 + P) {     // columns of the piece: dk
          const int lc = r0 - pc.col0;
          f4 k1 = {0.f, 0.f, 0.f, 0.f}, k2 = {0.f, 0.f, 0.f, 0.f};
          mma_tile<DOT_HIGHEST>(k1, tr(sDAq + pc.row0 * LT, LT).shift(r0, 0), rm(sQt, LD).shift(0, strip * 16), P);
          mma_tile<DOT_HIGHEST>(k2, tr(sDA + pc.row0 * LT, LT).shift(r0, 0), rm(sBt, LD).shift(0, strip * 16), P);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = r0 + tile_row(r), jl = lc + tile_row(r), d = dcol;
            const float cb = piece_col_leg(pc, sG, LD, j, d);
            const float x = scale * k1[r] + k2[r];
            bk[m][r] += x * cb;
            bgc[m][r] -= x * sKt[jl * LD + d];
          }
        }
      } else {
        // lean diagonal (b4.py:20-30): exact E = exp(clip(gc_i - gc_j, +-diff_clip))
        const float dc = cf.diff_clip;
        if (r0 >= pc.row0 && r0 < pc.row0 + P) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = r0 + tile_row(r), il = i - pc.row0, d = dcol;
            float sq = 0.f, sbk = 0.f;
            for (int jl = 0; jl < P; ++jl) {
              const int j = pc.col0 + jl;
              const float E = expf(fminf(fmaxf(sG[i * LD + d] - sG[j * LD + d], -dc), dc));
              const float ek = E * sKt[jl * LD + d];
              sq += sDAq[i * LT + j] * ek;
              sbk += sDA[i * LT + j] * ek;
            }
            const float x = scale * sq;
            bq[m][r] += x;
            bbk[m][r] += sbk;
            bgc[m][r] += sQt[il * LD + d] * x + sBt[il * LD + d] * sbk;
          }
        }
        if (r0 >= pc.col0 && r0 < pc.col0 + P) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = r0 + tile_row(r), jl = j - pc.col0, d = dcol;
            float s = 0.f;
            for (int il = 0; il < P; ++il) {
              const int i = pc.row0 + il;
              const float E = expf(fminf(fmaxf(sG[i * LD + d] - sG[j * LD + d], -dc), dc));
              const float M = sDAq[i * LT + j] * (scale * sQt[il * LD + d]) + sDA[i * LT + j] * sBt[il * LD + d];
              s += M * E;
            }
            bk[m][r] += s;
            bgc[m][r] -= sKt[jl * LD + d] * s;
          }
        }
      }
    }
  }
  __syncthreads();

  // dkb = A^T dWp, dwv = A^T dv_new (mega.py:42), the gate gradients dq3/dk3/db3/dgc3
  // (mega.py:45-51), and the combine with B4 (mega.py:52-59), tile by tile.
  load_rows<LD>(sX, a.dwp + tb, T, D, tid, NT);
  load_fragT<LD>(sY, a.dv_new_f + tb, D, T, 0, T, tid, NT);
  __syncthreads();
  f4 dgcT[NTW];
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    const int rt = St::rtile(wv, m);
    f4 dkb = {0.f, 0.f, 0.f, 0.f}, dwv = {0.f, 0.f, 0.f, 0.f};
    // A^T is upper triangular: rows of tile rt only see k >= 16*rt
    const int k0 = 16 * rt;
    mma_tile<B3>(dkb, tr(sA, LT).shift(16 * rt, k0), rm(sX, LD).shift(k0, strip * 16), T - k0);
    mma_tile<B3>(dwv, tr(sA, LT).shift(16 * rt, k0), rm(sY, LD).shift(k0, strip * 16), T - k0);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * rt + tile_row(r), d = dcol, e = i * D + d;
      const float ve = v[e], we = w[e], be = b[e], ke = k[e];
      a.dw[tb + e] = sanitize(dwv[r] * ve, clip);     // mega.py:57
      a.dv[tb + e] = sanitize(dwv[r] * we, clip);     // mega.py:58
      const float gi = sG[i * LD + d], gl = sG[(T - 1) * LD + d];
      const float egc = exp_nonpos(gi), ekg = exp_nonpos(gl - gi);
      const float mgc = gi < 0.f ? 1.f : 0.f, mkg = (gl - gi) < 0.f ? 1.f : 0.f;
      const float kb = (be * ke) * egc;
      const float kg = sanitize(ke * ekg, clip), qg = sanitize(q[e] * egc, clip);
      const float dqg = a.dqg[tb + e], dkg = a.dkg[tb + e];
      const float dx = dkg * kg;
      const float dq3 = dqg * egc;
      const float dk3 = (dkb[r] * egc) * be + dkg * ekg;
      const float db3 = (dkb[r] * egc) * ke;
      float dgc3 = ((dkb[r] * kb) * mgc + (dqg * qg) * mgc) - dx * mkg;
      dgc3 = sanitize(dgc3 + (i == T - 1 ? sCol[d] : 0.f), clip);
      const float dqv = sanitize(bq[m][r], clip);
      const float dbkv = sanitize(bbk[m][r], clip);
      const float dk4 = sanitize(bk[m][r] + dbkv * be, clip);
      const float db4 = sanitize(dbkv * ke, clip);
      const float dgc4 = sanitize(bgc[m][r], clip);
      a.dq[tb + e] = sanitize(dq3 + dqv, clip);
      a.dk[tb + e] = sanitize(dk3 + dk4, clip);
      a.db[tb + e] = sanitize(db3 + db4, clip);
      dgcT[m][r] = dgc3 + dgc4;
    }
  }
  __syncthreads();
  // B5: dg = reverse cumsum over the chunk rows of dgc3 + dgc4 (mega.py:53)
  float* sDgc = sX;
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    const int rt = St::rtile(wv, m);
#pragma unroll
    for (int r = 0; r < 4; ++r) sDgc[(16 * rt + tile_row(r)) * LD + dcol] = dgcT[m][r];
  }
  __syncthreads();
  {
    // reverse cumsum: column d split in NSEG runs of RUN rows
    constexpr int NSEG = NT / D, RUN = T / NSEG;
    const int d = tid % D, s = tid / D;
    float acc = 0.f;
    for (int i = RUN - 1; i >= 0; --i) {
      const int row = s * RUN + i;
      acc += sDgc[row * LD + d];
      sY[row * LD + d] = acc;
    }
    __syncthreads();
    float off = 0.f;
    for (int s2 = NSEG - 1; s2 > s; --s2) off += sY[(s2 * RUN) * LD + d];
    for (int i = 0; i < RUN; ++i) {
      const int row = s * RUN + i;
      a.dg[tb + row * D + d] = sanitize(sY[row * LD + d] + off, clip);
    }
  }
}

hipError_t launch_bwd_state(int D, const BwdStateArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((bwd_state_kernel<128, M>), dim3(a.n_chunks), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((bwd_state_kernel<64, M>), dim3(a.n_chunks), dim3(512), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_bwd_wy(int D, const BwdWyArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((bwd_wy_kernel<128, M>), dim3(a.n_chunks), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((bwd_wy_kernel<64, M>), dim3(a.n_chunks), dim3(512), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

}  // namespace gdn2
