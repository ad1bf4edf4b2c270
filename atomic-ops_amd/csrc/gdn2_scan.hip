// Sequential inter-chunk state scans of the GDN-2 operator (forward and reverse) on gfx950.
//
// One workgroup per (batch, head, 16-column slice of the value dimension): the recurrence is
// independent across value columns, so the D x 16 state slice is all a workgroup needs.
// The workgroup has D/16 waves; wave w keeps rows [16w, 16w+16) of the state slice in
// registers for the whole sequence, in the MFMA result layout (lane l holds rows
// 16w + 4(l/16) + e, e = 0..3, of column l%16).  With the k-permuted operand mapping of
// mma16 that layout is also the B-operand layout, so the state feeds the next chunk's
// products without any data movement.
//
// Products whose contraction runs over the key dimension (Wp h, Qg h, Kg dh) are split by
// key rows across waves: each wave multiplies with its own state rows and writes a 16x16
// partial tile per output row tile to LDS; a fixed-order sum over waves finishes them.
// Products over the chunk's time axis (Kg^T v_new, Aqk v_new, Qg^T dO, Wp^T dv_new) read
// v_new / dv_new (and dO) from transposed LDS slices with ds_read_b128.  A-operands stream
// from global memory as float4 (the WY kernel writes the transposed tiles Kg^T, Wp^T, Qg^T,
// Aqk^T, U^T for this) and are prefetched one chunk ahead into the second of two register
// sets; the chunk loop is unrolled by two so the sets never need copying, and all prefetch
// loads are unconditional so the compiler's vmcnt waits stay exact.  Per chunk: two
// workgroup barriers.
//
// Forward (fwd/cd_slim.py:12-30):  v_new = U - Wp h;  o = san(s Qg h + Aqk v_new);
//                                  h = san(e^gamma h + Kg^T v_new)
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

constexpr int LVT = T + 4;     // row stride of the transposed v_new slice [16][T]

template <int D>
struct FwdOps {
  float4 wp[4];    // Wp[16ti + r][16w + 4g .. +3]            ti = 0..3
  float4 qg[4];    // Qg[16ti + r][16w + 4g .. +3]
  float4 kg[4];    // Kg^T[16w + r][16u + 4g .. +3]           u = 0..3
  float4 aq[4];    // Aqk[16to + r][16u + 4g .. +3]           (used by the o-tile waves)
  float4 gm;       // gamma[16w + 4g .. +3]
  float4 uu;       // U^T[c0 + j_p][16t_p + 4g_p .. +3]       (v_new reduction pair)
};

template <int D, int MODE, bool RES>
__global__ __launch_bounds__(D / 16 * WAVE) void scan_fwd_kernel(ScanFwdArgs a) {
  constexpr int NW = D / 16, NT = NW * WAVE, NVB = D / 16, NP = 512 / NT;
  __shared__ float4 sPv[NW * 4 * WAVE];
  __shared__ float4 sPo[NW * 4 * WAVE];
  __shared__ float sVT[16 * LVT];
  __shared__ float4 sO1[4 * WAVE];
  const Cfg& cf = a.cfg;
  const float clip = cf.clip, scale = cf.scale;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int tid = threadIdx.x, l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  const bool o_role = NW == 8 ? (w >= 4) : true;
  const int to = NW == 8 ? (w >= 4 ? w - 4 : 0) : w;
  // the reduction pair of this thread: output tile tp, lane lp of its MFMA layout
  const int tp = (tid & 255) >> 6, lp = tid & 63, gp = lp >> 4, jp = lp & 15;

  f4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    h[e] = a.h0 ? a.h0[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] : 0.f;

  auto load = [&](FwdOps<D>& op, int c) {
    const size_t ch = (size_t)bh * nc + (c < nc ? c : nc - 1), tb = ch * T * D;
    const float* pw = a.wp + tb + (size_t)r * D + 16 * w + 4 * g;
    const float* pq = a.qg + tb + (size_t)r * D + 16 * w + 4 * g;
    const float* pk = a.kgT + tb + (size_t)(16 * w + r) * T + 4 * g;
    const float* pa = a.aqk + ch * T * T + (size_t)(16 * to + r) * T + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      op.wp[i] = ld4(pw + 16 * i * D);
      op.qg[i] = ld4(pq + 16 * i * D);
      op.kg[i] = ld4(pk + 16 * i);
      op.aq[i] = ld4(pa + 16 * i);
    }
    op.gm = ld4(a.gl + ch * D + 16 * w + 4 * g);
    op.uu = ld4(a.uT + tb + (size_t)(c0 + jp) * T + 16 * tp + 4 * gp);
  };

  auto step = [&](const FwdOps<D>& op, int c) {
    const size_t ch = (size_t)bh * nc + c, tb = ch * T * D;
    if constexpr (RES) {
#pragma unroll
      for (int e = 0; e < 4; ++e) a.h_pre[ch * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = h[e];
    }
    // partial Wp h and Qg h over this wave's 16 key rows
    const float4 hb = f4_to_float4(h);
    f4 pv[4], po[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      pv[ti] = f4{0.f, 0.f, 0.f, 0.f};
      po[ti] = f4{0.f, 0.f, 0.f, 0.f};
      mma16<MODE>(pv[ti], op.wp[ti], hb);
      mma16<MODE>(po[ti], op.qg[ti], hb);
    }
    drain(pv[0], pv[1], pv[2], pv[3]);
    drain(po[0], po[1], po[2], po[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      sPv[(w * 4 + ti) * WAVE + l] = f4_to_float4(pv[ti]);
      sPo[(w * 4 + ti) * WAVE + l] = f4_to_float4(po[ti]);
    }
    __syncthreads();
    // fixed-order reduction over waves: v_new = U - sum, O1 = sum
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int p = tid + q * NT, mat = p >> 8, pi = p & 255;
      const float4* src = mat ? sPo : sPv;
      float4 s = src[pi];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        const float4 x = src[w2 * 4 * WAVE + pi];
        s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
      }
      if (mat == 0) {
        const float4 vn = make_float4(op.uu.x - s.x, op.uu.y - s.y, op.uu.z - s.z, op.uu.w - s.w);
        st4(&sVT[jp * LVT + 16 * tp + 4 * gp], vn);
        if constexpr (RES) {
          float* pv2 = a.v_new + tb + (size_t)(16 * tp + 4 * gp) * D + c0 + jp;
          pv2[0] = vn.x; pv2[D] = vn.y; pv2[2 * D] = vn.z; pv2[3 * D] = vn.w;
        }
      } else {
        sO1[pi] = s;
      }
    }
    __syncthreads();
    float4 vt[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) vt[u] = ld4(&sVT[r * LVT + 16 * u + 4 * g]);
    f4 hn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) mma16<MODE>(hn, op.kg[u], vt[u]);
    if (o_role) {
      // straight-line over all 4 blocks: the blocks above the diagonal of Aqk are exact zeros
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 4; ++u) mma16<MODE>(acc, op.aq[u], vt[u]);
      drain(acc);
      const float4 o1 = sO1[to * WAVE + l];
      const float ov[4] = {o1.x, o1.y, o1.z, o1.w};
      float* po2 = a.o + tb + (size_t)(16 * to + 4 * g) * D + c0 + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) po2[e * D] = sanitize(scale * ov[e] + acc[e], clip);
    }
    drain(hn);
    const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = sanitize(h[e] * exp_nonpos(gmv[e]) + hn[e], clip);
  };

  FwdOps<D> A, B;
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
    const float* pk = a.kg + tb + (size_t)r * D + 16 * w + 4 * g;
    const float* pa = a.aqkT + ch * T * T + (size_t)(16 * ta + r) * T + 4 * g;
    const float* pq = a.qgT + tb + (size_t)(16 * w + r) * T + 4 * g;
    const float* pw = a.wpT + tb + (size_t)(16 * w + r) * T + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      op.kg[i] = ld4(pk + 16 * i * D);
      op.qgT[i] = ld4(pq + 16 * i);
      op.wpT[i] = ld4(pw + 16 * i);
    }
#pragma unroll
    for (int q = 0; q < PA; ++q) op.aqT[q] = ld4(pa + 16 * (ua + q));
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
#pragma unroll
    for (int e = 0; e < 4; ++e) a.dh_next[ch * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = dh[e];
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
      float* pv = a.dv_new + tb + (size_t)(16 * tp + 4 * gp) * D + c0 + jp;
      pv[0] = dv.x; pv[D] = dv.y; pv[2 * D] = dv.z; pv[3 * D] = dv.w;
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
  const bool res = a.h_pre != nullptr;
  dispatch_mode(a.cfg.dot_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) {
      if (res) hipLaunchKernelGGL((scan_fwd_kernel<128, M, true>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
      else hipLaunchKernelGGL((scan_fwd_kernel<128, M, false>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
    } else {
      if (res) hipLaunchKernelGGL((scan_fwd_kernel<64, M, true>), dim3(a.n_bh * 4), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((scan_fwd_kernel<64, M, false>), dim3(a.n_bh * 4), dim3(256), 0, s, a);
    }
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
