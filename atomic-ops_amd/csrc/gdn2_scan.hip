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
// over the chunk's time axis (Kg^T v_new, Wp^T dv_new) read v_new / dv_new from LDS in
// B-operand layout.  A-operands stream from global memory as one coalesced
// float4 per lane and block (fragment layout, written by the WY kernel) and are prefetched
// one chunk ahead into the second of two register sets; the chunk loop is unrolled by two so
// the sets never need copying, and all prefetch loads are unconditional so the compiler's
// vmcnt waits stay exact.  Per chunk: two workgroup barriers.
//
// Each scan carries only its chain (h -> v_new -> h, dh -> dv_new -> dh).  The forward output
// o, which needs h_pre and v_new but feeds nothing back, is computed chunk-parallel
// afterwards (gdn2_fwd.hip); the reverse scan's dO terms are computed chunk-parallel before it
// (gdn2_bwd.hip).
//
// Forward (fwd/cd_slim.py:12-30):  v_new = U - Wp h;  h = san(e^gamma h + Kg^T v_new)
// Reverse (bwd/mega.py:33-36):     dv_new = san(X + Kg dh);  dh = san(Y + e^gamma dh - Wp^T dv_new)
//                                  with X = Aqk^T dO, Y = Qg^T (s dO)
#include "gdn2_kernels.hpp"

namespace gdn2 {

// Workgroups of one (batch, head) land on the same XCD (blockIdx % 8 picks the XCD), so
// the chunk operands they all read are served from that XCD's L2.
__device__ __forceinline__ int xcd_remap(int nblk) {
  const int b = blockIdx.x;
  return (nblk % 8) ? b : (b % 8) * (nblk / 8) + b / 8;
}

struct FwdOps {
  float4 wp[4];    // FA(Wp) block (ti, w):    Wp[16ti + r][16w + 4g .. +3]
  float4 kg[4];    // FA(Kg^T) block (w, u):   Kg^T[16w + r][16u + 4g .. +3]
  float4 uu;       // FA(U^T) block (slice, tp), lane lp (the v_new reduction pair)
  float4 gm;       // gamma[16w + 4g .. +3]
};

// Prefetch loads for the next chunk are issued in small groups between the MFMA groups of the
// current one (sched_barrier keeps each group where it is written): a wave issuing a burst of
// loads stalls while the CU's vector memory path is busy, and with the loads spread out that
// stall overlaps the MFMAs already in flight.
#define GDN2_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

template <int D, int MODE>
__global__ __launch_bounds__(D / 16 * WAVE) void scan_fwd_kernel(ScanFwdArgs a) {
  constexpr int NW = D / 16, NVB = D / 16;
  __shared__ float4 sPv[NW * 4 * WAVE];    // partial (Wp h) tiles, [wave][ti][lane]
  __shared__ float4 sVB[4 * WAVE];         // v_new tiles in B-operand layout, [u][lane]
  const float clip = a.cfg.clip;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int tid = threadIdx.x, l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  // the reduction pair of this thread (threads < 256): output tile tp, lane lp
  const int tp = (tid & 255) >> 6, lp = tid & 63;
  const bool red = tid < 4 * WAVE;

  f4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    h[e] = a.h0 ? a.h0[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] : 0.f;

  auto base = [&](int c) { return (size_t)bh * nc + (c < nc ? c : nc - 1); };   // clamped chunk
  auto load_all = [&](FwdOps& op, int c) {
    const size_t tb = base(c) * T * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      op.wp[i] = ld4(a.wp_f + tb + frag_blk(i, w, D) + 4 * l);
      op.kg[i] = ld4(a.kgT_f + tb + frag_blk(w, i, T) + 4 * l);
    }
    op.uu = ld4(a.uT_f + tb + frag_blk(vb, tp, T) + 4 * lp);
    op.gm = ld4(a.gl + base(c) * D + 16 * w + 4 * g);
  };

  // one chunk step on `op`; prefetches chunk cn into `nx`
  auto step = [&](const FwdOps& op, int c, FwdOps& nx, int cn) {
    const size_t ch = (size_t)bh * nc + c, tb = ch * T * D;
    const size_t tbn = base(cn) * T * D;
    stg4(a.h_pre_f + ch * D * D + frag_blk(vb, w, D) + 4 * l, f4_to_float4(h));
    // partial Wp h over this wave's 16 key rows
    const float4 hb = f4_to_float4(h);
    f4 pv[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      pv[ti] = f4{0.f, 0.f, 0.f, 0.f};
      mma16<MODE>(pv[ti], op.wp[ti], hb);
      GDN2_SCHED_FENCE();
      nx.wp[ti] = ld4(a.wp_f + tbn + frag_blk(ti, w, D) + 4 * l);
      GDN2_SCHED_FENCE();
    }
    drain(pv[0], pv[1], pv[2], pv[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) sPv[(w * 4 + ti) * WAVE + l] = f4_to_float4(pv[ti]);
    __syncthreads();
    // fixed-order reduction over waves: v_new = U - sum
    if (red) {
      float4 s = sPv[tid];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) s = add4(s, sPv[w2 * 4 * WAVE + tid]);
      const float4 vn = sub4(op.uu, s);
      sVB[tid] = vn;
      stg4(a.v_new_f + tb + frag_blk(vb, tp, T) + 4 * lp, vn);
    }
    nx.uu = ld4(a.uT_f + tbn + frag_blk(vb, tp, T) + 4 * lp);
    nx.gm = ld4(a.gl + base(cn) * D + 16 * w + 4 * g);
    __syncthreads();
    // the B operands are read before the chain: the fences below would otherwise hold each
    // LDS read back until the previous MFMA has issued
    float4 vb4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) vb4[u] = sVB[u * WAVE + l];
    f4 hn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      mma16<MODE>(hn, op.kg[u], vb4[u]);
      GDN2_SCHED_FENCE();
      nx.kg[u] = ld4(a.kgT_f + tbn + frag_blk(w, u, T) + 4 * l);
      GDN2_SCHED_FENCE();
    }
    drain(hn);
    const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = sanitize(h[e] * exp_nonpos(gmv[e]) + hn[e], clip);
  };

  FwdOps A, B;
  load_all(A, 0);
  int c = 0;
  for (; c + 1 < nc; c += 2) {
    step(A, c, B, c + 1);
    step(B, c + 1, A, c + 2);
  }
  if (c < nc) step(A, c, B, c + 1);
#pragma unroll
  for (int e = 0; e < 4; ++e) a.hf[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = h[e];
}

// Lane lt of block u of a FA(X^T) tile set in LDS (xs[u][lane], X of T x 16 columns) ->
// lane lt of block u of FA(X): X[16 u + r][4 g .. 4 g + 3] is lane 4 g + e + 16 (r / 4),
// component r % 4 of xs[u].
__device__ __forceinline__ float4 frag_transpose_lds(const float4* xs, int u, int lt) {
  const float* f = reinterpret_cast<const float*>(xs + u * WAVE);
  const int rr = lt & 15, gg = lt >> 4, c = 16 * (rr >> 2), e = rr & 3;
  return make_float4(f[4 * (4 * gg + c) + e], f[4 * (4 * gg + 1 + c) + e], f[4 * (4 * gg + 2 + c) + e],
                     f[4 * (4 * gg + 3 + c) + e]);
}

struct BwdOps {
  float4 kg[4];    // FA(Kg) block (ti, w):    Kg[16ti + r][16w + 4g .. +3]
  float4 wpT[4];   // FA(Wp^T) block (w, u):   Wp^T[16w + r][16u + 4g .. +3]
  float4 xx;       // FA(X^T) block (slice, tp), lane lp: X = Aqk^T dO (the dv_new reduction pair)
  float4 yy;       // FA(Y^T) block (slice, w): Y = s Qg^T dO, this lane's 4 state rows
  float4 gm;       // gamma[16w + 4g .. +3]
};

// Reverse scan, chain only: the dO terms X = Aqk^T dO and Y = s Qg^T dO do not depend on dh and
// come precomputed per chunk (bwd_pre_kernel).
template <int D, int MODE>
__global__ __launch_bounds__(D / 16 * WAVE) void scan_bwd_kernel(ScanBwdArgs a) {
  constexpr int NW = D / 16, NVB = D / 16;
  __shared__ float4 sP[NW * 4 * WAVE];     // partial (Kg dh) tiles, [wave][ti][lane]
  __shared__ float4 sDB[4 * WAVE];         // dv_new tiles in B-operand layout, [u][lane]
  __shared__ __attribute__((aligned(16))) float sTr[NW * 16 * TRP];   // per-wave transpose tiles
  const float clip = a.cfg.clip;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int tid = threadIdx.x, l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  const int tp = (tid & 255) >> 6, lp = tid & 63;
  const bool red = tid < 4 * WAVE;

  f4 dh;
#pragma unroll
  for (int e = 0; e < 4; ++e) dh[e] = a.dhf[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r];

  // step s processes chunk nc-1-s; steps past the last are clamped to chunk 0 (loads only)
  auto chunk = [&](int s) { return (size_t)bh * nc + (s < nc ? nc - 1 - s : 0); };
  auto load_all = [&](BwdOps& op, int s) {
    const size_t ch = chunk(s), tb = ch * T * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      op.kg[i] = ld4(a.kg_f + tb + frag_blk(i, w, D) + 4 * l);
      op.wpT[i] = ld4(a.wpT_f + tb + frag_blk(w, i, T) + 4 * l);
    }
    op.xx = ld4(a.x_f + tb + frag_blk(vb, tp, T) + 4 * lp);
    op.yy = ld4(a.y_f + ch * D * D + frag_blk(vb, w, D) + 4 * l);
    op.gm = ld4(a.gl + ch * D + 16 * w + 4 * g);
  };

  auto step = [&](const BwdOps& op, int s, BwdOps& nx, int sn) {
    const size_t ch = chunk(s), tb = ch * T * D;
    const size_t chn = chunk(sn), tbn = chn * T * D;
    const float4 db = f4_to_float4(dh);
    f4 p[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      p[ti] = f4{0.f, 0.f, 0.f, 0.f};
      mma16<MODE>(p[ti], op.kg[ti], db);
      GDN2_SCHED_FENCE();
      nx.kg[ti] = ld4(a.kg_f + tbn + frag_blk(ti, w, D) + 4 * l);
      GDN2_SCHED_FENCE();
    }
    // dh entering this chunk's step (mega.py:35) as FA(dh_next) block (w, slice)
    const float4 dhv = wave_transpose16(sTr + w * 16 * TRP, db, r, g);
    drain(p[0], p[1], p[2], p[3]);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) sP[(w * 4 + ti) * WAVE + l] = f4_to_float4(p[ti]);
    __syncthreads();
    // dv_new = san(Aqk^T dO + Kg dh): fixed-order sum over waves, then the dO term
    if (red) {
      float4 sm = sP[tid];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) sm = add4(sm, sP[w2 * 4 * WAVE + tid]);
      const float4 dv = san4(add4(op.xx, sm), clip);
      sDB[tid] = dv;
    }
    nx.xx = ld4(a.x_f + tbn + frag_blk(vb, tp, T) + 4 * lp);
    nx.yy = ld4(a.y_f + chn * D * D + frag_blk(vb, w, D) + 4 * l);
    nx.gm = ld4(a.gl + chn * D + 16 * w + 4 * g);
    __syncthreads();
    float4 db4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) db4[u] = sDB[u * WAVE + l];
    f4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      mma16<MODE>(z, op.wpT[u], db4[u]);
      GDN2_SCHED_FENCE();
      nx.wpT[u] = ld4(a.wpT_f + tbn + frag_blk(w, u, T) + 4 * l);
      GDN2_SCHED_FENCE();
    }
    float4 dvv = db;
    if (red) dvv = frag_transpose_lds(sDB, tp, lp);     // FA(dv_new) block (tp, slice)
    drain(z);
    const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
    const float yv[4] = {op.yy.x, op.yy.y, op.yy.z, op.yy.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) dh[e] = sanitize((yv[e] + dh[e] * exp_nonpos(gmv[e])) - z[e], clip);
    // stores last: the next step's waits for the prefetch loads above then do not also cover them
    stg4(a.dh_next_f + ch * D * D + frag_blk(w, vb, D) + 4 * l, dhv);
    if (red) stg4(a.dv_new_f + tb + frag_blk(tp, vb, D) + 4 * lp, dvv);
  };

  BwdOps A, B;
  load_all(A, 0);
  int s = 0;
  for (; s + 1 < nc; s += 2) {
    step(A, s, B, s + 1);
    step(B, s + 1, A, s + 2);
  }
  if (s < nc) step(A, s, B, s + 1);
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
