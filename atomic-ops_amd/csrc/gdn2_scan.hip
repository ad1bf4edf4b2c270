// Sequential inter-chunk state scans of the GDN-2 operator (forward and reverse) on gfx950.
//
// One workgroup per (batch, head, 16-column slice of the value dimension): the recurrence is
// independent across value columns, so the D x 16 state slice is all a workgroup needs.
// The workgroup has D/16 waves; wave w keeps rows [16w, 16w+16) of the state slice in
// registers for the whole sequence, in the MFMA result layout (lane l holds rows
// 16w + 4(l/16) + e, e = 0..3, of column l%16).  With the k-permuted operand mapping of
// mma16 that layout is also the B-operand layout, so the state feeds the next chunk's
// products without any data movement, and it is lane l of block (slice, w) of the
// transposed state in fragment layout, so saving it is one float4 store per lane.
//
// Products whose contraction runs over the key dimension (Wp h, Kg dh) are split by key
// rows across waves: each wave multiplies with its own state rows and writes a 16x16 partial
// tile per output row tile to LDS; a fixed-order sum over waves finishes them.  Products
// over the chunk's time axis (Kg^T v_new, Wp^T dv_new, Aqk^T dO, Qg^T dO) read v_new / dv_new
// / dO from LDS in B-operand layout.  A-operands stream from global memory as one coalesced
// float4 per lane and block (fragment layout, written by the WY kernel) and are prefetched
// one chunk ahead into the second of two register sets; the chunk loop is unrolled by two so
// the sets never need copying, and all prefetch loads are unconditional so the compiler's
// vmcnt waits stay exact.  Per chunk: two workgroup barriers.
//
// The forward scan carries only the chain h -> v_new -> h; the output o, which needs h_pre
// and v_new but feeds nothing back, is computed chunk-parallel afterwards (gdn2_fwd.hip).
//
// Forward (fwd/cd_slim.py:12-30):  v_new = U - Wp h;  h = san(e^gamma h + Kg^T v_new)
// Reverse (bwd/mega.py:33-36):     dv_new = san(Aqk^T dO + Kg dh);
//                                  dh = san(Qg^T (s dO) + e^gamma dh - Wp^T dv_new)
#include "gdn2_kernels.hpp"

namespace gdn2 {

// Workgroups of one (batch, head) land on the same XCD (blockIdx % 8 picks the XCD), so
// the chunk operands they all read are served from that XCD's L2.
__device__ __forceinline__ int xcd_remap(int nblk) {
  const int b = blockIdx.x;
  return (nblk % 8) ? b : (b % 8) * (nblk / 8) + b / 8;
}

constexpr int LVT = T + 4;     // row stride of the transposed dO / dv_new slices [16][T]

struct FwdOps {
  float4 wp[4];    // FA(Wp) block (ti, w):    Wp[16ti + r][16w + 4g .. +3]
  float4 kg[4];    // FA(Kg^T) block (w, u):   Kg^T[16w + r][16u + 4g .. +3]
  float4 uu;       // FA(U^T) block (slice, tp), lane lp (the v_new reduction pair)
  float4 gm;       // gamma[16w + 4g .. +3]
};

template <int D, int MODE>
__global__ __launch_bounds__(D / 16 * WAVE) void scan_fwd_kernel(ScanFwdArgs a) {
  constexpr int NW = D / 16, NT = NW * WAVE, NVB = D / 16;
  __shared__ float4 sPv[NW * 4 * WAVE];    // partial (Wp h) tiles, [wave][ti][lane]
  __shared__ float4 sVB[4 * WAVE];         // v_new tiles in B-operand layout, [u][lane]
  const float clip = a.cfg.clip;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int tid = threadIdx.x, l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  // the reduction pair of this thread (threads < 256): output tile tp, lane lp
  const int tp = (tid & 255) >> 6, lp = tid & 63;

  f4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    h[e] = a.h0 ? a.h0[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] : 0.f;

  auto load = [&](FwdOps& op, int c) {
    const size_t ch = (size_t)bh * nc + (c < nc ? c : nc - 1), tb = ch * T * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      op.wp[i] = ld4(a.wp_f + tb + frag_blk(i, w, D) + 4 * l);
      op.kg[i] = ld4(a.kgT_f + tb + frag_blk(w, i, T) + 4 * l);
    }
    op.uu = ld4(a.uT_f + tb + frag_blk(vb, tp, T) + 4 * lp);
    op.gm = ld4(a.gl + ch * D + 16 * w + 4 * g);
  };

  auto step = [&](const FwdOps& op, int c) {
    const size_t ch = (size_t)bh * nc + c, tb = ch * T * D;
    st4(a.h_pre_f + ch * D * D + frag_blk(vb, w, D) + 4 * l, f4_to_float4(h));
    // partial Wp h over this wave's 16 key rows
    const float4 hb = f4_to_float4(h);
    f4 pv[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      pv[ti] = f4{0.f, 0.f, 0.f, 0.f};
      mma16<MODE>(pv[ti], op.wp[ti], hb);
    }
    drain(pv[0], pv[1], pv[2], pv[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) sPv[(w * 4 + ti) * WAVE + l] = f4_to_float4(pv[ti]);
    __syncthreads();
    // fixed-order reduction over waves: v_new = U - sum
    if (tid < 4 * WAVE) {
      float4 s = sPv[tid];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) s = add4(s, sPv[w2 * 4 * WAVE + tid]);
      const float4 vn = sub4(op.uu, s);
      sVB[tid] = vn;
      st4(a.v_new_f + tb + frag_blk(vb, tp, T) + 4 * lp, vn);
    }
    __syncthreads();
    f4 hn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) mma16<MODE>(hn, op.kg[u], sVB[u * WAVE + l]);
    drain(hn);
    const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = sanitize(h[e] * exp_nonpos(gmv[e]) + hn[e], clip);
  };

  FwdOps A, B;
  load(A, 0);
  int c = 0;
  for (; c + 1 < nc; c += 2) {
    load(B, c + 1);
    step(A, c);
    load(A, c + 2);
    step(B, c + 1);
  }
  if (c < nc) step(A, c);
#pragma unroll
  for (int e = 0; e < 4; ++e) a.hf[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = h[e];
}

template <int D>
struct BwdOps {
  float4 kg[4];              // Kg[16ti + r][16w + 4g .. +3]         ti = 0..3
  float4 aqT[16 / (D / 16)]; // Aqk^T[16ta + r][16u + 4g .. +3]      for this wave's (ta, u) pairs
  float4 qgT[4];             // Qg^T[16w + r][16u + 4g .. +3]
  float4 wpT[4];             // Wp^T[16w + r][16u + 4g .. +3]
  float4 gm;
};

template <int D, int MODE>
__global__ __launch_bounds__(D / 16 * WAVE) void scan_bwd_kernel(ScanBwdArgs a) {
  constexpr int NW = D / 16, NT = NW * WAVE, NVB = D / 16, PA = 16 / NW;
  __shared__ float4 sP[NW * 4 * WAVE];
  __shared__ float sDVT[16 * LVT];
  __shared__ float sDOT[2][16 * LVT];        // dO slice of the chunk, transposed, double-buffered
  const Cfg& cf = a.cfg;
  const float clip = cf.clip, scale = cf.scale;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int tid = threadIdx.x, l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  const int ta = (w * PA) / 4, ua = (w * PA) % 4;    // Aqk^T dO pairs (ta, ua .. ua+PA-1)
  const int tp = (tid & 255) >> 6, lp = tid & 63, gp = lp >> 4, jp = lp & 15;
  // dO staging: thread t < 256 moves dO[t/4][c0 + 4(t%4) .. +3] of a chunk
  const int srow = (tid & 255) >> 2, scol = 4 * (tid & 3);

  f4 dh;
#pragma unroll
  for (int e = 0; e < 4; ++e) dh[e] = a.dhf[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r];

  // step s processes chunk nc-1-s; loads for a step past the last are clamped (unused)
  auto chunk = [&](int s) { return (size_t)bh * nc + (s < nc ? nc - 1 - s : 0); };
  auto load = [&](BwdOps<D>& op, int s) {
    const size_t ch = chunk(s), tb = ch * T * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      op.kg[i] = ld4(a.kg_f + tb + frag_blk(i, w, D) + 4 * l);
      op.qgT[i] = ld4(a.qgT_f + tb + frag_blk(w, i, T) + 4 * l);
      op.wpT[i] = ld4(a.wpT_f + tb + frag_blk(w, i, T) + 4 * l);
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) op.aqT[q] = ld4(a.aqkT_f + ch * T * T + frag_blk(ta, ua + q, T) + 4 * l);
    op.gm = ld4(a.gl + ch * D + 16 * w + 4 * g);
  };
  auto load_do = [&](int s) { return ld4(a.dout + chunk(s) * T * D + (size_t)srow * D + c0 + scol); };
  auto stage_do = [&](int buf, const float4& x) {
    if (tid < 256) {
      sDOT[buf][(scol + 0) * LVT + srow] = x.x;
      sDOT[buf][(scol + 1) * LVT + srow] = x.y;
      sDOT[buf][(scol + 2) * LVT + srow] = x.z;
      sDOT[buf][(scol + 3) * LVT + srow] = x.w;
    }
  };

  auto step = [&](const BwdOps<D>& op, int s) {
    const int buf = s & 1;
    const size_t ch = chunk(s), tb = ch * T * D;
    const float4 dnext = load_do(s + 1);           // dO of the next step, staged below
    // dh entering this chunk's step (mega.py:35)
    st4(a.dh_next_f + ch * D * D + frag_blk(vb, w, D) + 4 * l, f4_to_float4(dh));
    float4 dob[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) dob[u] = ld4(&sDOT[buf][r * LVT + 16 * u + 4 * g]);
    const float4 db = f4_to_float4(dh);
    f4 p[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      p[ti] = f4{0.f, 0.f, 0.f, 0.f};
      mma16<MODE>(p[ti], op.kg[ti], db);
    }
    // this wave's share of Aqk^T dO (partial tile ta); dO blocks picked with compile-time indices
    f4 pa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < PA; ++q) {
      float4 dsel = dob[0];
#pragma unroll
      for (int u = 1; u < 4; ++u)
        if (u == ua + q) dsel = dob[u];
      mma16<MODE>(pa, op.aqT[q], dsel);
    }
    // Qg^T (s dO) for the own rows
    f4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) mma16<MODE>(y, op.qgT[u], scale4(dob[u], scale));
    drain(p[0], p[1], p[2], p[3]);
    drain(pa, y);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      float4 x = f4_to_float4(p[ti]);
      if (ti == ta) { x.x += pa[0]; x.y += pa[1]; x.z += pa[2]; x.w += pa[3]; }
      sP[(w * 4 + ti) * WAVE + l] = x;
    }
    __syncthreads();
    if (tid < 256) {
      float4 sm = sP[tid];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        const float4 x = sP[w2 * 4 * WAVE + tid];
        sm.x += x.x; sm.y += x.y; sm.z += x.z; sm.w += x.w;
      }
      const float4 dv = make_float4(sanitize(sm.x, clip), sanitize(sm.y, clip), sanitize(sm.z, clip),
                                    sanitize(sm.w, clip));
      st4(&sDVT[jp * LVT + 16 * tp + 4 * gp], dv);
      st4(a.dv_new_f + tb + frag_blk(vb, tp, T) + 4 * lp, dv);
    }
    stage_do(buf ^ 1, dnext);
    __syncthreads();
    f4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) mma16<MODE>(z, op.wpT[u], ld4(&sDVT[r * LVT + 16 * u + 4 * g]));
    drain(z);
    const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) dh[e] = sanitize((y[e] + dh[e] * exp_nonpos(gmv[e])) - z[e], clip);
  };

  stage_do(0, load_do(0));
  BwdOps<D> A, B;
  load(A, 0);
  __syncthreads();
  int s = 0;
  for (; s + 1 < nc; s += 2) {
    load(B, s + 1);
    step(A, s);
    load(A, s + 2);
    step(B, s + 1);
  }
  if (s < nc) step(A, s);
#pragma unroll
  for (int e = 0; e < 4; ++e) a.dh0[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = dh[e];
}

hipError_t launch_scan_fwd(int D, const ScanFwdArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.dot_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((scan_fwd_kernel<128, M>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((scan_fwd_kernel<64, M>), dim3(a.n_bh * 4), dim3(256), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_scan_bwd(int D, const ScanBwdArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((scan_bwd_kernel<128, M>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((scan_bwd_kernel<64, M>), dim3(a.n_bh * 4), dim3(256), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

}  // namespace gdn2
