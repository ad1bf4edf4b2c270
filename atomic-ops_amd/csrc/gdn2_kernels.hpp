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
// kind 2: as kind 1 for a diagonal block wider than the 64-token part (bs2 = 128 / 256): r and
//         gc[s1-1] are the block's first and last rows, which lie in other parts; they come
//         expressed in this part's gc frame from the anchor buffer (anchor_kernel).
// Pieces are P x P squares, P = min(bs2, 32); P = 8 (bs2 = 8) is narrower than an MFMA tile
// and such pieces are formed per element.
struct Piece {
  int8_t row0, col0, P, kind, anchor, s0, s1, pad;
};
constexpr int MAX_PIECES = 40;     // bs2 = 8 at T = 64: 36 pieces
struct PieceList {
  Piece p[MAX_PIECES];
  int n;
};
// A Piece read field by field, also from the kernel argument block seen in its own address
// space (kernarg_fresh), where the implicit copy does not apply.
template <typename P>
__device__ __forceinline__ Piece load_piece(const P& s) {
  Piece p;
  p.row0 = s.row0;
  p.col0 = s.col0;
  p.P = s.P;
  p.kind = s.kind;
  p.anchor = s.anchor;
  p.s0 = s.s0;
  p.s1 = s.s1;
  p.pad = s.pad;
  return p;
}

struct Cfg {
  float scale, wy_eps, ome, clip, diff_clip;   // ome = 1 - wy_eps, rounded once on the host
  int diag, dot_mode, solve_mode, b3_mode, mb;
  int nc;        // chunks per (batch, head) sequence of this segment
  int seq_ld;    // tokens between consecutive (batch, head) sequences of the raw operator tensors
  // group = G in {2, 4}: the operator's chunk is bt = 64 G with wy_eps > 0, run as G parts of
  // 64 tokens (part j = chunk c with c % G == j).  The WY inverse of the big chunk is block
  // lower triangular; its diagonal blocks are the parts' own inverses (I + (1-eps) Akk_jj)^-1,
  // and forward substitution over the blocks gives, exactly, part j = the 64-chunk form whose
  // erase term reads the damped state h_d(j) instead of the state h(j) entering the part:
  //   h(0) = h_d(0) = the state entering the big chunk,
  //   h(j+1) = e^gamma_j h(j) + Kg_j^T v_new_j,   h_d(j+1) = e^gamma_j h_d(j) + (1-eps) Kg_j^T v_new_j
  // (the cross-part scores are carried by the states; only the erase term sees the damping).
  // The output and the carried state use h.  Equivalently h_d(j) = h(j) - eps Delta(j) with
  // Delta(0) = 0, Delta(j+1) = e^gamma_j Delta(j) + Kg_j^T v_new_j, so the backward adds to the
  // undamped form the cotangent of Delta: EZ(j) = eps Wp_j^T dv_new_j + e^gamma_j EZ(j+1)
  // (j >= 1, EZ(G) = 0), which reaches part j-1's Kg^T v_new term and, through the decay,
  // gamma_j's gradient (sum_v EZ(j+1) Delta(j)).  group = 1: no damping across parts (with
  // wy_eps = 0 every chunk size is the 64-chunk operator).
  int group;
  PieceList pieces;
  // the piece that covers 16 x 16 score tile (ti, tj), at [4 ti + tj], for ti >= tj (pieces are
  // squares of side 16 or 32 on multiples of their side, so a tile lies in exactly one).  32-bit
  // entries: a kernel reads them with a wave-uniform index as scalar loads (there is no scalar
  // byte load, and a vector load of kernel arguments would make its wait cover every memory
  // operation in flight).
  int32_t tile_piece[16];
};

// Piece i of a piece list held in the kernel arguments, read as two scalar dwords (i wave-uniform)
__device__ __forceinline__ Piece piece_at(const PieceList& pl, int i) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&pl.p[i]);
  const uint32_t w0 = w[0], w1 = w[1];
  Piece p;
  p.row0 = (int8_t)(w0 & 0xff);
  p.col0 = (int8_t)((w0 >> 8) & 0xff);
  p.P = (int8_t)((w0 >> 16) & 0xff);
  p.kind = (int8_t)(w0 >> 24);
  p.anchor = (int8_t)(w1 & 0xff);
  p.s0 = (int8_t)((w1 >> 8) & 0xff);
  p.s1 = (int8_t)((w1 >> 16) & 0xff);
  p.pad = (int8_t)(w1 >> 24);
  return p;
}

// Offset in floats of a chunk (index (b, h) * nc + chunk of the segment) in a raw operator
// tensor -- q..g, o, dO and the input gradients, (B, H, seq_ld, D) with the segment starting at
// the pointer passed in.  Per-segment buffers (residual, workspace) are chunk-contiguous.
template <int D, typename C>
__device__ __forceinline__ size_t io_off(const C& c, int chunk) {
  const int bh = chunk / c.nc, cc = chunk - bh * c.nc;
  return ((size_t)bh * c.seq_ld + (size_t)cc * T) * D;
}

// Per-chunk outputs of the WY build.  "_f" outputs are in fragment layout (gdn2_common.hpp):
//   wp_f FA(Wp) (T x D), uT_f FA(U^T) (D x T), kg_f FA(Kg) (T x D),
//   qg_f FA(Qg) (T x D), aqk_f FA(Aqk) (T x T).  A (T x T) and gl (D) are row-major.  The plain
//   row-major
//   aqk / akk / wp / u / kg / qg are written only for the stage-level entry point.  Any
//   pointer may be null (not written).
struct WyFwdArgs {
  const void *q, *k, *v, *w, *b, *g;   // fp32, or bfloat16 bits for the bf16-input variant
  const float* anc;    // kind-2 pieces: the anchor buffer (AnchorArgs), else null
  float *wp_f, *uT_f, *kg_f, *qg_f, *aqk_f;
  float *A, *gl;
  float *aqk, *akk, *wp, *u, *kg, *qg;
  int n_chunks;
  int g_is_gc;     // nonzero: g holds the in-chunk cumulative sum gc itself (the stage entry points)
  Cfg cfg;
};

// Checkpoint blocks of the selective recompute (state_ckpt = K): per (batch, head) the nc chunks
// are cut into nfull = nc / K blocks of K chunks, then the R = nc % K chunks left over: into
// blocks of S = Cfg::group chunks (one chunk each without damping; R is a multiple of S, since
// nc and K are) when that makes at most two blocks, else into one block of R.  Every block
// starts from a stored checkpoint (slot j of nblk per (batch, head)) and the backward steps the
// state through it.  The short remainder blocks keep the backward's grid within one round: at
// K = 3 and nc = 32 one remainder block of two chunks per (batch, head) needed 16 workgroups
// more than the chip holds at once, which started only when the first blocks finished, while
// single-chunk blocks dispatched after the full ones run in the slots that finish first (at the
// cost of one more checkpoint).  K <= 1: every chunk is a block of its own.
struct CkptBlocks {
  int K, RL, nfull, nblk;    // RL: length of a remainder block
  __host__ __device__ CkptBlocks(int nc, int K_, int S) : K(K_ > 1 ? K_ : 1), RL(1), nfull(0), nblk(0) {
    nfull = nc / K;
    const int R = nc - nfull * K;
    const int s = K_ > 1 ? S : 1;
    RL = R == 0 ? 1 : (R / s <= 2 ? s : R);
    nblk = nfull + R / RL;
  }
  __host__ __device__ int start(int j) const { return j < nfull ? j * K : nfull * K + (j - nfull) * RL; }
  __host__ __device__ int len(int j) const { return j < nfull ? K : RL; }
  // the checkpoint slot of chunk c (its block's index when c starts a block), else -1
  __host__ __device__ int slot(int c) const {
    if (c < nfull * K) return c % K == 0 ? c / K : -1;
    const int r = c - nfull * K;
    return r % RL == 0 ? nfull + r / RL : -1;
  }
};

// Forward state scan: reads FA(Wp), FA(Kg), FA(U^T), gl; writes the final state hf
// (row-major D x D) and, when h_pre_f / v_new_f are set, per chunk the entering state h_pre as
// FA(h_pre^T) (D x D) and v_new as FA(v_new^T) (D x T).  With o set it also reads FA(Qg),
// FA(Aqk) and writes o (row-major T x D per chunk); otherwise out_fwd computes o.
// h_pre_f keeps the state entering the first chunk of each checkpoint block (CkptBlocks of
// ckpt and Cfg::group), at its slot of nblk per (batch, head); ckpt 0 or 1: every chunk's.
// reset (may be null): one byte per (batch, head) and chunk, row (b, h) of nc bytes; nonzero =
// the state entering that chunk is zero (a document boundary at the chunk's first token; at
// chunk 0 it replaces h0).
struct ScanFwdArgs {
  const float *wp_f, *kg_f, *uT_f, *gl, *h0, *qg_f, *aqk_f;
  float *hf, *o, *h_pre_f, *v_new_f;    // o, h_pre_f, v_new_f may be null
  int nc, n_bh, ckpt;
  Cfg cfg;
  const uint8_t* reset;
};

// Chunk-parallel output: o = san(s Qg h_pre + Aqk v_new), o row-major (T x D per chunk).
struct OutFwdArgs {
  const float *qg_f, *aqk_f, *h_pre_f, *v_new_f;
  float* o;
  int n_chunks;
  Cfg cfg;
};

// The reverse scan's dO terms, chunk-parallel: X = Aqk^T dO as FA(X^T) (D x T) and
// Y = s Qg^T dO as FA(Y^T) (D x D), from FA(Aqk), FA(Qg) and dO (row-major).
struct BwdPreArgs {
  const float *aqk_f, *qg_f, *dout;
  float *x_f, *y_f;
  int n_chunks;
  Cfg cfg;
};

// Reverse state scan: reads FA(Wp), FA(Kg), gl, X, Y; writes dv_new as FA(dv_new) (T x D),
// dh_next as FA(dh_next) (D x D), dh0 row-major.
// With Cfg::group = G > 1 the cotangent of the damping correction of each part j >= 1 reaches
// part j - 1's Kg v_new term (EZ, Cfg::group): added to dh there, and written per part as
// FA(ez) (D x D, the dh_next layout) for bwd_state_rc's dKg.
struct ScanBwdArgs {
  const float *wp_f, *kg_f, *gl, *x_f, *y_f, *dhf;
  float *dv_new_f, *dh_next_f, *dh0, *ez_f;
  int nc, n_bh;
  Cfg cfg;
};

// Reads FA(dv_new) (T x D), FA(v_new^T) (D x T), FA(h_pre^T), FA(dh_next) (D x D) and dO
// (row-major);
// dqg / dwp / dkg are (T x D) per chunk, written as FA(dqg^T) / FA(dwp^T) / FA(dkg^T).
struct BwdStateArgs {
  const float *dout, *dv_new_f, *v_new_f, *h_pre_f, *dh_next_f;
  float *dqg, *dwp, *dkg, *dlast;
  int n_chunks;
  Cfg cfg;
};

// bwd_state with the states recomputed from checkpoints: per (batch, head) checkpoint block
// (CkptBlocks) the state entering the block (checkpoint FA(h^T), nblk per (batch, head)) is
// stepped forward through the block, h <- san(e^gamma h + Kg^T v_new), from FA(Kg), gl and the
// stored FA(v_new^T) -- the forward scan's own update, bit for bit -- and each chunk's
// reductions use it as h_pre.  Outputs as BwdStateArgs.
struct BwdStateRcArgs {
  const float *dout, *dv_new_f, *v_new_f, *hck_f, *dh_next_f, *kg_f, *gl, *ez_f;
  float *dqg, *dwp, *dkg, *dlast;
  int nc, n_bh, ckpt;
  Cfg cfg;
};

struct BwdWyArgs {
  const float *q, *k, *v, *w, *b, *g, *A, *dout, *v_new_f, *dv_new_f;
  const float* anc;    // kind-2 pieces: the anchor buffer (AnchorArgs), else null
  const float *dqg, *dwp, *dkg, *dlast;
  float *dq, *dk, *dv, *dw, *db, *dg;
  int n_chunks;
  Cfg cfg;
};

// Token recurrence for serving (gdn2_decode.hip): n_tok tokens per (batch, head) in order.
// q..g (and o) at ((b H + h) seq_ld + t) D + d, fp32 or bfloat16 bits (in_bf16 / out_bf16);
// state_in / state_out (B, H, D, D) row-major (key, value) in the state dtype (state_bf16),
// state_in null = zero state, state_out may equal state_in; reset: null or B x n_tok bytes,
// nonzero = zero state entering that token of batch row b; fuse: q, k l2-normalised, b, w
// sigmoid, g = -exp(a_log[h]) softplus(g + dt_bias[d]) in the kernel; cap: per-head Frobenius
// cap tau on the state.
struct DecodeArgs {
  const void *q, *k, *v, *w, *b, *g;
  const float *a_log, *dt_bias;
  const uint8_t* reset;
  const void* state_in;
  void *o, *state_out;
  int H, n_tok, seq_ld;
  int in_bf16, out_bf16, state_bf16, fuse, cap;
  float scale, tau;
};

hipError_t launch_decode(int D, const DecodeArgs& a, int n_bh, hipStream_t s);

// Anchors of the diagonal blocks wider than a 64-token part (bs2 = 64 B, B = 2 or 4 parts; kind-2
// pieces): for part j of a block, in the part's own gc frame (gc restarts at every part),
//   anc[(part, 0, d)] = gc of the block's first row  = gc_0[0][d] - sum_{i<j} gl_i[d],
//   anc[(part, 1, d)] = gc of the block's last row   = sum_{i>=j} gl_i[d],
// with gl_i the last row of part i's gc, all formed with chunk_cumsum's arithmetic (so gl_i is
// bit-identical to what every other kernel computes) and the sums in ascending part order.
struct AnchorArgs {
  const void* g;       // fp32 or bfloat16 bits
  float* anc;          // (n_chunks, 2, D)
  int n_chunks, B;     // B parts per diagonal block
  Cfg cfg;
};
hipError_t launch_anchors(int D, const AnchorArgs& a, hipStream_t s, bool bf16_inputs);

hipError_t launch_wy_fwd(int D, const WyFwdArgs& a, hipStream_t s, bool bf16_inputs = false);

// Grid of a persistent kernel (one workgroup per CU, each walking chunks blockIdx.x,
// + gridDim.x, ...): min(n_chunks, CUs of the current device).
inline hipError_t persistent_grid(int n_chunks, dim3* grid) {
  int dev = 0, ncu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  if (ncu < 1) return hipErrorInvalidDevice;
  *grid = dim3(n_chunks < ncu ? n_chunks : ncu);
  return hipSuccess;
}
hipError_t launch_scan_fwd(int D, const ScanFwdArgs& a, hipStream_t s);
hipError_t launch_out_fwd(int D, const OutFwdArgs& a, hipStream_t s);
hipError_t launch_bwd_pre(int D, const BwdPreArgs& a, hipStream_t s);
hipError_t launch_scan_bwd(int D, const ScanBwdArgs& a, hipStream_t s);
hipError_t launch_bwd_state(int D, const BwdStateArgs& a, hipStream_t s);
hipError_t launch_bwd_state_rc(int D, const BwdStateRcArgs& a, hipStream_t s);
hipError_t launch_bwd_wy(int D, const BwdWyArgs& a, hipStream_t s);

// Diagnostics: C[M,N] = A[M,K] * B[K,N] (row-major, fp32 storage) through the MFMA tile
// routine of the given dot mode.  M, N, K multiples of 16, at most 64 x 64 x 128.
hipError_t launch_gemm_probe(int mode, const float* A, const float* B, float* C, int M, int N,
                             int K, hipStream_t s);
// Diagnostics: stream n4 float4s (a multiple of 256): mode 0 copy src -> dst, 1 read src,
// 2 fill dst.
hipError_t launch_stream_probe(int mode, const void* src, void* dst, size_t n4, hipStream_t s);
// Diagnostics: blocks workgroups of four waves, each wave iters rounds of eight independent
// mma16 (4 v_mfma_f32_16x16x4_f32 each); out[blocks * 256] gets each lane's accumulator sum
// (512 iters).
hipError_t launch_mfma_probe(int blocks, int iters, float* out, hipStream_t s);

// Linear work index of this workgroup such that consecutive indices (workgroups of one
// (batch, head), which read the same chunk operands) land on the same XCD (blockIdx % 8 picks
// the XCD) and are served from that XCD's L2.  Identity unless nblk % 8 == 0.
__device__ __forceinline__ int xcd_remap(int nblk) {
  const int b = blockIdx.x;
  return (nblk % 8) ? b : (b % 8) * (nblk / 8) + b / 8;
}

// Leg factors of a score piece from gc values (fwd/scores.py:16-22, 39-65): gi / gj the gc of
// the row / column, ga the anchor's (kind 0) or the diagonal block's first row (kinds 1, 2), gz
// the block's last row (kinds 1, 2).  The forward's MFMA path inlines the same formulas.
__device__ __forceinline__ float leg_row(int kind, float gi, float ga, float gz) {
  if (kind == 0) return fast_exp(min0(gi - ga));
  const float half = 0.5f * (ga - gz);
  return fast_exp((gi - ga) + half);
}
__device__ __forceinline__ float leg_col(int kind, float gj, float ga, float gz) {
  if (kind == 0) return fast_exp(min0(ga - gj));
  const float half = 0.5f * (ga - gz);
  return fast_exp((ga - gj) - half);
}
// The same with gc in a row-major LDS tile (ld LD); ar / az: channel d's values of the anchor
// buffer (kind 2; unused otherwise).
__device__ __forceinline__ float piece_ga(const Piece& pc, const float* sG, int LD, int d, float ar) {
  return pc.kind == 2 ? ar : sG[(pc.kind == 0 ? pc.anchor : pc.s0) * LD + d];
}
__device__ __forceinline__ float piece_gz(const Piece& pc, const float* sG, int LD, int d, float az) {
  return pc.kind == 2 ? az : pc.kind == 1 ? sG[(pc.s1 - 1) * LD + d] : 0.f;
}
__device__ __forceinline__ float piece_row_leg(const Piece& pc, const float* sG, int LD, int i, int d, float ar,
                                               float az) {
  return leg_row(pc.kind, sG[i * LD + d], piece_ga(pc, sG, LD, d, ar), piece_gz(pc, sG, LD, d, az));
}
__device__ __forceinline__ float piece_col_leg(const Piece& pc, const float* sG, int LD, int j, int d, float ar,
                                               float az) {
  return leg_col(pc.kind, sG[j * LD + d], piece_ga(pc, sG, LD, d, ar), piece_gz(pc, sG, LD, d, az));
}

}  // namespace gdn2
