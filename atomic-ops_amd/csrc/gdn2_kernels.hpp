// Kernel argument blocks and launch declarations shared by the HIP kernels and the C-ABI.
#pragma once
#include "gdn2_common.hpp"

namespace gdn2 {

// One square piece of the T x T score matrix computed with a single pair of rescaling legs.
// kind 0: off-diagonal piece, legs exp(min(gc_i - gc_a, 0)) / exp(min(gc_a - gc_j, 0))
//         with anchor row a.
// kind 1: diagonal-block piece of block [s0, s1): BTL legs exp(gc_i - r + half) and
//         exp(r - gc_j - half), r = gc[s0], half = (gc[s0] - gc[s1-1]) / 2; or, with the
//         lean diagonal, the exact exp(clip(gc_i - gc_j, +-diff_clip)) per element.
struct Piece {
  int8_t row0, col0, P, kind, anchor, s0, s1, pad;
};
constexpr int MAX_PIECES = 16;
struct PieceList {
  Piece p[MAX_PIECES];
  int n;
};

struct Cfg {
  float scale, wy_eps, ome, clip, diff_clip;   // ome = 1 - wy_eps, rounded once on the host
  int diag, dot_mode, solve_mode, b3_mode, mb;
  PieceList pieces;
};

// Per-chunk outputs of the WY build.  Row-major tiles are (T x D) / (T x T); the "T"
// variants are the same tiles transposed, (D x T) / (T x T), written for the scans so that
// all their A-operands are contiguous float4 loads.  Any pointer may be null (not written).
struct WyFwdArgs {
  const float *q, *k, *v, *w, *b, *g;
  float *aqk, *aqkT, *A, *wp, *wpT, *u, *uT, *kg, *kgT, *qg, *qgT, *gl;
  float* akk;          // masked, sanitized Akk (before the (1-eps) factor)
  int n_chunks;        // B*H*nc
  Cfg cfg;
};

struct ScanFwdArgs {
  const float *wp, *uT, *kgT, *qg, *gl, *aqk, *h0;
  float *o, *hf, *h_pre, *v_new;   // h_pre / v_new null for a forward-only call
  int nc, n_bh;
  Cfg cfg;
};

struct ScanBwdArgs {
  const float *wpT, *kg, *qgT, *gl, *aqkT, *dout, *dhf;
  float *dv_new, *dh_next, *dh0;
  int nc, n_bh;
  Cfg cfg;
};

struct BwdStateArgs {
  const float *dout, *dv_new, *v_new, *h_pre, *dh_next;
  float *dqg, *dwp, *dkg, *dlast;
  int n_chunks;
  Cfg cfg;
};

struct BwdWyArgs {
  const float *q, *k, *v, *w, *b, *g, *A, *aqk, *dout, *v_new, *dv_new;
  const float *dqg, *dwp, *dkg, *dlast;
  float *dq, *dk, *dv, *dw, *db, *dg;
  int n_chunks;
  Cfg cfg;
};

hipError_t launch_wy_fwd(int D, const WyFwdArgs& a, hipStream_t s);
hipError_t launch_scan_fwd(int D, const ScanFwdArgs& a, hipStream_t s);
hipError_t launch_scan_bwd(int D, const ScanBwdArgs& a, hipStream_t s);
hipError_t launch_bwd_state(int D, const BwdStateArgs& a, hipStream_t s);
hipError_t launch_bwd_wy(int D, const BwdWyArgs& a, hipStream_t s);

// Diagnostics: C[M,N] = A[M,K] * B[K,N] (row-major, fp32 storage) through the MFMA tile
// routine of the given dot mode.  M, N, K multiples of 16, at most 64 x 64 x 128.
hipError_t launch_gemm_probe(int mode, const float* A, const float* B, float* C, int M, int N,
                             int K, hipStream_t s);

// Device-side leg factors of a score piece (used by the forward scores and by B4).
__device__ __forceinline__ float piece_row_leg(const Piece& pc, const float* sG, int LD, int i, int d) {
  const float gi = sG[i * LD + d];
  if (pc.kind == 0) return exp_nonpos(gi - sG[pc.anchor * LD + d]);
  const float r = sG[pc.s0 * LD + d];
  const float half = 0.5f * (r - sG[(pc.s1 - 1) * LD + d]);
  return expf((gi - r) + half);
}
__device__ __forceinline__ float piece_col_leg(const Piece& pc, const float* sG, int LD, int j, int d) {
  const float gj = sG[j * LD + d];
  if (pc.kind == 0) return exp_nonpos(sG[pc.anchor * LD + d] - gj);
  const float r = sG[pc.s0 * LD + d];
  const float half = 0.5f * (r - sG[(pc.s1 - 1) * LD + d]);
  return expf((r - gj) - half);
}

}  // namespace gdn2
