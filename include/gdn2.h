/*
 * gdn2.h -- C ABI of the MI355X (gfx950) GDN-2 operator library `libgdn2_hip.so`.
 *
 * This is the drop-in boundary under the Python API `make_blr_trainable(cfg, scale)`.
 * Plain pointers and sizes only: every tensor argument is a device pointer to a float32
 * buffer (contiguous, except that the raw operator tensors of a segment may lie inside longer
 * sequences, see gdn2_desc.seq_ld), and `stream` is a `hipStream_t` (NULL = the default stream).  Kernels are
 * enqueued on `stream`; no call synchronises the device, allocates memory or keeps a
 * pointer after it returns (except the profiling calls, see below).  Every entry point
 * returns a gdn2_status; on failure gdn2_last_error() describes the problem.
 *
 * Layouts (head-major, as in the reference; a chunk is `bt` consecutive tokens):
 *   q, k, v, w, b, g, o, dq .. dg   (B, H, L, D)      == (B, H, nc, bt, D), nc = L / bt
 *   h0, h_final, dh_final, dh0      (B, H, D, D)      rows = key channel, cols = value channel
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   gdn2_fwd  : the custom_vjp forward of one segment, `_fwd` + `core_fwd`
 *               (atomic_gdn2/pipeline.py:20-36), i.e. build_scores (fwd/scores.py:87-97),
 *               wy_solve_leafbatched (fwd/solve.py:51-59) and recompute_and_scan_slim
 *               (fwd/cd_slim.py:34-51).
 *   gdn2_bwd  : the custom_vjp backward of one segment, `core_bwd` (pipeline.py:38-47),
 *               i.e. backward_mega (bwd/mega.py:61-79) before `_fin`.
 *   gdn2_wy_stage : the chunk-parallel stages alone (scores, WY inverse, W/U recompute),
 *               for stage-level checks (fwd/scores.py:87, fwd/solve.py:51, cd_slim.py:17-21).
 *   gdn2_scores : build_scores itself, gc given (fwd/scores.py:87-97).
 */
#ifndef GDN2_H_
#define GDN2_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN2_ABI_VERSION 3

/* Matmul precision modes (atomic_gdn2/precision.py:27-31; config.py:41-43). */
enum { GDN2_DOT_HIGHEST = 0, GDN2_DOT_BF16X3 = 1, GDN2_DOT_DEFAULT = 2 };
/* Diagonal-block treatment of the scores (config.py:46). */
enum { GDN2_DIAG_BTL = 0, GDN2_DIAG_LEAN = 1 };
/* Status codes. */
enum { GDN2_OK = 0, GDN2_ERR_INVALID = 1, GDN2_ERR_UNSUPPORTED = 2, GDN2_ERR_HIP = 3 };

/* One segment call.  Field meaning follows BLRConfig (atomic_gdn2/config.py:29-50).
 * Supported by this build: bt in {64, 128, 256} (128 and 256 as 2 and 4 parts of 64 tokens;
 * with wy_eps > 0 they need state_ckpt >= 1), D in {64, 128}, L % bt == 0, bs2 >= 8 (so one of
 * 8, 16, ..., 256), bs2 | score_bs | bt, mb a power of two dividing bt.  bs2 = 8 forms the
 * scores per element; bs2 = 128 / 256 (a BTL diagonal block wider than a 64-token part) adds a
 * pre-pass that writes each part's block end rows into the workspace (kernel id 9).
 *   L        tokens of this segment (a multiple of bt).
 *   seq_ld   tokens between the starts of consecutive (b, h) sequences in the raw operator
 *            tensors q..g, o, d_o, dq..dg (0 = L, i.e. contiguous (B, H, L, D)).  A segment
 *            [t0, t0 + L) of a (B, H, L_full, D) tensor is passed as the pointer advanced by
 *            t0 * D floats with seq_ld = L_full: the kernels read and write it in place, the way
 *            the reference's segment loop slices and concatenates (pipeline.py:57-64).
 *   state_ckpt  how the residual keeps the state for the backward (no counterpart in the
 *            reference, whose residual keeps the state entering every chunk, pipeline.py:25):
 *            0 = the state entering every chunk; K >= 1 = only the state entering each
 *            checkpoint block (blocks of K chunks, see HPRE below), the backward recomputes the
 *            others. */
typedef struct gdn2_desc {
  int32_t B, H, L, D;
  int32_t bt, score_bs, bs2, mb;
  int32_t diag, dot_mode, solve_dot_mode, b3_dot_mode;
  int32_t seq_ld, state_ckpt;
  double scale, wy_eps, clip, diff_clip;
} gdn2_desc;

/* Residual buffer written by gdn2_fwd and read by gdn2_bwd: sub-buffers at the offsets
 * reported by gdn2_residual_layout (bytes, 256-aligned), float32.  Whatever bt is, the kernels
 * work on parts of 64 tokens (bt = 128 / 256 is 2 / 4 consecutive parts), so every per-chunk
 * entry below is per 64-token part: n64 = L / 64 parts per (b, h) of the segment, p = part.
 *   AQK   (B,H,n64, 64*64)  gated q.k scores of the part, FRAG(Aqk)            (pipeline.py:25)
 *   A     (B,H,n64,64,64)   the part's own WY inverse (I + (1-eps) Akk_pp)^-1, row-major; at
 *                           bt = 64 the reference's A, at bt > 64 the diagonal blocks of the
 *                           reference's bt x bt inverse (the off-diagonal blocks are carried
 *                           by the states, gdn2_kernels.hpp Cfg::group)         (pipeline.py:25)
 *   HPRE  (B,H,nck, D*D)    state entering each part (nck = n64, state_ckpt 0 or 1) or only
 *                           the first part of each checkpoint block (state_ckpt = K: parts
 *                           0, K, .., K (n64 / K - 1), then the n64 % K parts left over as one
 *                           block, or as blocks of bt / 64 parts -- single parts without
 *                           damping -- when those are at most two), FRAG(h_pre^T) (cd_slim.py:23)
 *   VNEW  (B,H,n64, D*64)   v_new of each part, FRAG(v_new^T)                  (cd_slim.py:29)
 *   WP    (B,H,n64, 64*D)   W = A (b k e^gc) of each part, FRAG(W)              (cd_slim.py:18)
 *   KG    (B,H,n64, 64*D)   gated k, FRAG(Kg)                                   (cd_slim.py:22)
 *   QG    (B,H,n64, 64*D)   gated q, FRAG(Qg)                                   (cd_slim.py:22)
 *   GL    (B,H,n64,D)       gc (within the part) of the part's last row         (cd_slim.py:20)
 * FRAG(M) of an R x C matrix M is the MFMA fragment order the kernels load with one
 * coalesced float4 per lane: 16x16 blocks in row-major block order (C/16 blocks per block
 * row, 256 floats each); inside a block, floats [4 l, 4 l + 4) with l = r + 16 c hold
 * M[16 bi + r][16 bj + 4 c + e], e = 0..3 (r = 0..15, c = 0..3). */
enum { GDN2_RES_AQK = 0, GDN2_RES_A, GDN2_RES_HPRE, GDN2_RES_VNEW, GDN2_RES_WP, GDN2_RES_KG,
       GDN2_RES_QG, GDN2_RES_GL, GDN2_RES_COUNT };

int gdn2_abi_version(void);
const char* gdn2_last_error(void);

/* Validates `d` and reports the residual sub-buffer offsets and total size in bytes. */
int gdn2_residual_layout(const gdn2_desc* d, size_t offsets[GDN2_RES_COUNT], size_t* total_bytes);
/* Workspace sizes in bytes (0 on an invalid descriptor). */
size_t gdn2_fwd_workspace_bytes(const gdn2_desc* d, int with_residual);
size_t gdn2_bwd_workspace_bytes(const gdn2_desc* d);

/* Forward of one segment.  h0 may be NULL (zero state).  residual may be NULL for a
 * forward-only call (nothing is kept for a backward pass); otherwise it must hold
 * gdn2_residual_layout() bytes.  workspace holds gdn2_fwd_workspace_bytes(d, residual!=NULL). */
int gdn2_fwd(const gdn2_desc* d, const float* q, const float* k, const float* v, const float* w,
             const float* b, const float* g, const float* h0, float* o, float* h_final,
             void* residual, void* workspace, void* stream);

/* Forward of one segment with bfloat16 inputs (raw bf16 bits, same layouts): q..g are widened
 * to fp32 on load; state, accumulation and outputs are fp32 exactly as in gdn2_fwd, which this
 * equals bit for bit on the same (bf16-representable) values.  For the forward-only
 * long-context path (bf16 activations, fp32 state carried between calls through h0/h_final):
 * the forward half of make_blr_trainable (atomic_gdn2/pipeline.py:51-64) called with bf16
 * inputs, without the up-front cast to fp32.  residual may be NULL (no backward). */
int gdn2_fwd_bf16(const gdn2_desc* d, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                  const uint16_t* w, const uint16_t* b, const uint16_t* g, const float* h0, float* o,
                  float* h_final, void* residual, void* workspace, void* stream);

/* Forward-only prefill with document resets at chunk granularity: gdn2_fwd without a residual,
 * q..g fp32 (in_dtype 0) or bfloat16 bits (in_dtype 1, as gdn2_fwd_bf16), and chunk_reset NULL
 * or one byte per (batch, head, 64-token chunk), row (b*H + h) of L/64 bytes: nonzero = the
 * state entering that chunk is zero (its first token starts a new document; at chunk 0 it
 * replaces h0).  Replaces the chunkwise part of chunk_forward_inference in the reference's
 * inference module (notebooks/gdn2_v031_stage2_tpu.ipynb, cell 1, INFERENCE_V031: the
 * _cd_inference_body call with per-row segment resets).  At bt = 128 / 256 with wy_eps > 0 a
 * reset on a 64-token part that does not start a bt chunk zeroes the damped state with the
 * true one, so the remaining parts of that chunk run as a damped chunk of their own (the
 * reference's inference API places document starts only at bt boundaries, and
 * atomic_gdn2.inference flags only those).  workspace holds gdn2_fwd_workspace_bytes(d, 0). */
int gdn2_fwd_reset(const gdn2_desc* d, int in_dtype, const void* q, const void* k, const void* v,
                   const void* w, const void* b, const void* g, const float* h0,
                   const uint8_t* chunk_reset, float* o, float* h_final, void* workspace,
                   void* stream);

/* Token recurrence for serving (no MFMA; see gdn2_decode). */
typedef struct gdn2_decode_desc {
  int32_t B, H, D;        /* D in {64, 128} */
  int32_t n_tok;          /* tokens per (batch, head), >= 1, processed in order */
  int32_t seq_ld;         /* tokens between consecutive (b,h) rows of q..g and o, >= n_tok */
  int32_t in_dtype;       /* q..g: 0 fp32, 1 bfloat16 bits */
  int32_t out_dtype;      /* o: 0 fp32, 1 bfloat16 bits */
  int32_t state_dtype;    /* state_in / state_out: 0 fp32, 1 bfloat16 bits */
  int32_t fuse_prologue;  /* 1: q, k raw (l2-normalised), b, w logits (sigmoid), g the raw
                           * gate: g = -exp(a_log[h]) * softplus(g + dt_bias[d]) */
  int32_t cap;            /* 1: cap the state's per-head Frobenius norm at stability_tau */
  double scale;
  double stability_tau;
} gdn2_decode_desc;

/* n_tok tokens of the recurrence per (batch, head): decode_step of the reference's inference
 * module (INFERENCE_V031 decode_step / _decode_body) for n_tok = 1, and n_tok consecutive
 * decode_step calls (the tail of chunk_forward_inference) otherwise.  q..g and o are
 * (B, H, seq_ld, D) (element (b,h,t,d) at ((b*H + h)*seq_ld + t)*D + d; decode_step's (B,H,D)
 * tensors are seq_ld = n_tok = 1); state_in / state_out (B, H, D, D) (key, value) in the state
 * dtype; state_in NULL = zero state; state_out may equal state_in.  reset NULL or B*n_tok bytes
 * (row b): nonzero = the state entering that token of batch row b is zero.  a_log (H) and
 * dt_bias (D) are read only with fuse_prologue.  Per token: S = reset ? 0 : state;
 * h = diag(e^min(g,0)) S; v_new = w*v - h^T (b*k); h += k v_new^T; o = h^T (scale*q); with cap,
 * h *= min(1, tau / max(||h||_F, 1e-12)); NaN and +-Inf in h and o become 0; the state is
 * rounded to the state dtype after every token, o to the output dtype. */
int gdn2_decode(const gdn2_decode_desc* d, const void* q, const void* k, const void* v,
                const void* w, const void* b, const void* g, const float* a_log,
                const float* dt_bias, const uint8_t* reset, const void* state_in, void* o,
                void* state_out, void* stream);

/* Forward of one segment without a residual, like gdn2_fwd(d, ..., residual = NULL, ...), with
 * the workspace in a fixed 64 MiB (67108864-byte) device array inside the library instead of
 * a caller buffer.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It calls no allocating routine.  Calls whose gdn2_fwd_workspace_bytes(d, 0)
 * exceeds 64 MiB (e.g. more than 453 chunks of B*H*L/bt at D = 128) fail with
 * GDN2_ERR_UNSUPPORTED.  Every call on one GPU shares that GPU's array: calls that overlap in
 * time on one GPU (different streams or host threads) race; serialise them.  Nothing in the
 * array needs clearing: each call writes every byte it reads. */
int gdn2_fwd_noalloc(const gdn2_desc* d, const float* q, const float* k, const float* v,
                     const float* w, const float* b, const float* g, const float* h0, float* o,
                     float* h_final, void* stream);

/* Backward of one segment: cotangents d_o (B,H,L,D) and d_hf (B,H,D,D) -> the raw
 * (sanitized at cfg.clip) gradients of q, k, v, w, b, g and h0, all float32. */
int gdn2_bwd(const gdn2_desc* d, const float* q, const float* k, const float* v, const float* w,
             const float* b, const float* g, const void* residual, const float* d_o,
             const float* d_hf, float* dq, float* dk, float* dv, float* dw, float* db, float* dg,
             float* dh0, void* workspace, void* stream);

/* Chunk-parallel forward stages only, all outputs row-major: aqk, akk, A (B,H,nc,bt,bt);
 * wp, u, kg, qg (B,H,nc,bt,D); gl (B,H,nc,D).  akk and A may be NULL.  akk is the masked,
 * sanitized Akk before the (1 - wy_eps) factor; A is the sanitized inverse. */
int gdn2_wy_stage(const gdn2_desc* d, const float* q, const float* k, const float* v,
                  const float* w, const float* b, const float* g, float* aqk, float* akk,
                  float* A, float* wp, float* u, float* kg, float* qg, float* gl, void* stream);

/* Kernel A alone with the reference's signature: build_scores(q, k, b, gc, scale, cfg) ->
 * (Aqk, Akk) (atomic_gdn2/fwd/scores.py:87-97).  gc (B,H,L,D) is the caller's in-chunk
 * cumulative gate (cumsum of g within each 64-token chunk), used as given; aqk, akk
 * (B,H,nc,64,64) row-major, masked and sanitized, akk before the (1 - wy_eps) factor.
 * bt == 64 only (the scores of a chunk of 64 tokens). */
int gdn2_scores(const gdn2_desc* d, const float* q, const float* k, const float* b, const float* gc,
                float* aqk, float* akk, void* stream);

/* Diagnostics: C[M,N] = A[M,K] B[K,N] (row-major float32) through the kernels' MFMA tile
 * routine in the given dot mode.  M, N <= 64, K <= 128, all multiples of 16. */
int gdn2_debug_gemm(int mode, const float* A, const float* B, float* C, int M, int N, int K,
                    void* stream);

/* Diagnostics (no counterpart in the reference): the HBM streaming rate that the kernels' byte
 * counts are judged against.  mode 0 copies `bytes` from src to dst, 1 reads src (dst: at least
 * 16 bytes, written only on a sentinel sum), 2 fills dst; one float4 per thread, bytes a positive
 * multiple of 4096, both buffers 16-byte aligned. */
int gdn2_debug_stream(int mode, const void* src, void* dst, size_t bytes, void* stream);

/* Diagnostics (no counterpart in the reference): the sustained fp32 MFMA rate that the kernels'
 * FLOP counts are judged against.  `blocks` workgroups of four waves; every wave issues `iters`
 * rounds of eight independent 16-deep products, each four dependent v_mfma_f32_16x16x4_f32
 * (8192 FLOP) as the kernels issue them, i.e. the launch does blocks * 4 * iters * 8 * 8192 FLOP.
 * out holds blocks * 256 floats; each is 512 * iters (the lane's accumulator sum for all-ones
 * operands).  1 <= blocks, iters <= 1 << 20. */
int gdn2_debug_mfma(int blocks, int iters, float* out, void* stream);

/* Per-kernel timing with HIP events recorded on the launch stream around every kernel.
 * gdn2_prof_begin(n) starts recording for up to n launches (process-wide, not re-entrant);
 * gdn2_prof_end synchronises on the recorded events and returns, per kernel id, the summed
 * duration in milliseconds and the launch count, then stops recording.
 * Kernel ids: 0 wy_fwd, 1 scan_fwd (with the output unless state_ckpt == 0 in training),
 * 2 scan_bwd, 3 bwd_state (state_ckpt == 0), 4 bwd_wy, 5 out_fwd (training, state_ckpt == 0),
 * 6 bwd_pre, 7 bwd_state_rc (state_ckpt >= 1: bwd_state with the states recomputed), 8 decode,
 * 9 anchors (bs2 > 64: the diagonal blocks' end rows, before wy_fwd and bwd_wy). */
#define GDN2_NUM_KERNELS 10
int gdn2_prof_begin(int max_launches);
int gdn2_prof_end(double ms_sum[GDN2_NUM_KERNELS], int counts[GDN2_NUM_KERNELS]);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_H_ */
