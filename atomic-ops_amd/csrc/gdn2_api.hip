// C ABI of the GDN-2 library: descriptor validation, residual / workspace layout, kernel
// sequencing per segment, and optional per-kernel HIP-event timing.
#include <mutex>
#include <string>
#include <vector>

#include "../../include/gdn2.h"
#include "gdn2_kernels.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

gdn2::Cfg make_cfg(const gdn2_desc* d);

// Validation mirrors BLRConfig.__post_init__ (atomic_gdn2/config.py:52-65) plus this
// build's supported geometry.
int validate(const gdn2_desc* d) {
  if (!d) return fail(GDN2_ERR_INVALID, "null descriptor");
  if (d->B <= 0 || d->H <= 0 || d->L <= 0 || d->D <= 0) return fail(GDN2_ERR_INVALID, "non-positive shape");
  if (d->bt <= 0 || d->L % d->bt) return fail(GDN2_ERR_INVALID, "L must be divisible by bt");
  if (d->score_bs <= 0 || d->bs2 <= 0 || d->bt % d->score_bs || d->score_bs % d->bs2)
    return fail(GDN2_ERR_INVALID, "need bt % score_bs == 0 and score_bs % bs2 == 0");
  if (!pow2(d->mb) || d->bt % d->mb || !pow2(d->bt / d->mb))
    return fail(GDN2_ERR_INVALID, "mb and bt/mb must be powers of two dividing bt");
  if (!(d->wy_eps >= 0.0 && d->wy_eps < 1.0)) return fail(GDN2_ERR_INVALID, "wy_eps in [0,1)");
  for (int m : {d->dot_mode, d->solve_dot_mode, d->b3_dot_mode})
    if (m < GDN2_DOT_HIGHEST || m > GDN2_DOT_DEFAULT) return fail(GDN2_ERR_INVALID, "unknown dot mode");
  if (d->diag != GDN2_DIAG_BTL && d->diag != GDN2_DIAG_LEAN) return fail(GDN2_ERR_INVALID, "unknown diag");
  if (!(d->clip > 0.0)) return fail(GDN2_ERR_INVALID, "clip must be positive");
  // bt = 128 / 256 run as 2 / 4 parts of 64 tokens (Cfg::group); without damping every chunk
  // size is the 64-token operator
  if (d->bt != gdn2::T && d->bt != 2 * gdn2::T && d->bt != 4 * gdn2::T)
    return fail(GDN2_ERR_UNSUPPORTED, "this build supports bt in {64, 128, 256}");
  if (d->D != 64 && d->D != 128) return fail(GDN2_ERR_UNSUPPORTED, "this build supports D in {64, 128}");
  if (d->bs2 < 8) return fail(GDN2_ERR_UNSUPPORTED, "this build supports bs2 >= 8");
  if (d->seq_ld != 0 && d->seq_ld < d->L) return fail(GDN2_ERR_INVALID, "seq_ld must be 0 or >= L");
  if (d->state_ckpt < 0) return fail(GDN2_ERR_INVALID, "state_ckpt must be >= 0");
  // the score pieces partition the lower triangle, so every 16 x 16 tile on or below the
  // diagonal has one (the kernels index the piece list with Cfg::tile_piece)
  const gdn2::Cfg c = make_cfg(d);
  for (int t = 0; t < 16; ++t)
    if (t / 4 >= t % 4 && c.tile_piece[t] < 0) return fail(GDN2_ERR_UNSUPPORTED, "score tile without a piece");
  return GDN2_OK;
}

// Calls that keep or use a residual: validate() plus the residual's own constraint.
int validate_residual(const gdn2_desc* d) {
  const int st = validate(d);
  if (st) return st;
  if (d->bt > gdn2::T && d->wy_eps > 0.0 && d->state_ckpt == 0)
    return fail(GDN2_ERR_UNSUPPORTED, "bt >= 128 with wy_eps > 0 needs state_ckpt >= 1");
  return GDN2_OK;
}

// bt = 128 / 256 run as 2 / 4 parts of 64 tokens (gdn2_kernels.hpp, Cfg::group).  With
// wy_eps > 0 the backward's state recompute needs every part of a big chunk in one block, so
// the checkpoint interval (in 64-token chunks) is rounded up to a multiple of the group.
int damped_group(const gdn2_desc* d) { return d->wy_eps > 0.0 ? d->bt / gdn2::T : 1; }
int eff_ckpt(const gdn2_desc* d) {
  const int k = d->state_ckpt;
  const int G = damped_group(d);
  return (G > 1 && k % G) ? k + (G - k % G) : k;
}

// Pieces of the two-level block-local rescaling (fwd/scores.py:39-72): for each row block
// [q0, q0+bs2) of outer block p0: its diagonal block, the level-2 part [p0, q0) with anchor
// q0 and the level-1 part [0, p0) with anchor p0, cut into squares of side min(bs2, 32).  A
// diagonal block wider than the part (bs2 > T) covers the whole part: kind-2 pieces, whose
// block ends come from the anchor buffer.
void make_pieces(int T, int sbs, int bs2, gdn2::PieceList* out) {
  const int P = bs2 < 32 ? bs2 : 32;
  int n = 0;
  auto add = [&](int r, int c, int kind, int anchor, int s0, int s1) {
    gdn2::Piece& p = out->p[n++];
    p.row0 = (int8_t)r; p.col0 = (int8_t)c; p.P = (int8_t)P; p.kind = (int8_t)kind;
    p.anchor = (int8_t)anchor; p.s0 = (int8_t)s0; p.s1 = (int8_t)s1; p.pad = 0;
  };
  if (bs2 > T) {
    for (int r = 0; r < T; r += P)
      for (int c = 0; c <= r; c += P) add(r, c, 2, 0, 0, 0);
    out->n = n;
    return;
  }
  for (int q0 = 0; q0 < T; q0 += bs2) {
    const int q1 = q0 + bs2, p0 = (q0 / sbs) * sbs;
    for (int r = q0; r < q1; r += P)
      for (int c = q0; c <= r; c += P) add(r, c, 1, q0, q0, q1);
    for (int c = p0; c < q0; c += P)
      for (int r = q0; r < q1; r += P) add(r, c, 0, q0, 0, 0);
    for (int c = 0; c < p0; c += P)
      for (int r = q0; r < q1; r += P) add(r, c, 0, p0, 0, 0);
  }
  out->n = n;
}

gdn2::Cfg make_cfg(const gdn2_desc* d) {
  gdn2::Cfg c{};
  c.scale = (float)d->scale;
  c.wy_eps = (float)d->wy_eps;
  c.ome = (float)(1.0 - d->wy_eps);
  c.clip = (float)d->clip;
  c.diff_clip = (float)d->diff_clip;
  c.diag = d->diag;
  c.dot_mode = d->dot_mode;
  c.solve_mode = d->solve_dot_mode;
  c.b3_mode = d->b3_dot_mode;
  c.mb = d->mb < gdn2::T ? d->mb : gdn2::T;    // leaves inside a 64-token (half) chunk
  c.nc = d->L / gdn2::T;
  c.seq_ld = d->seq_ld ? d->seq_ld : d->L;
  c.group = damped_group(d);
  // the score pieces inside one 64-token (half) chunk: at bt = 128 the pieces of the 128
  // geometry that lie inside a half are the 64 geometry's with the outer block capped at 64
  // (the pieces crossing the halves are carried by the state, see Cfg::group)
  make_pieces(gdn2::T, d->score_bs < gdn2::T ? d->score_bs : gdn2::T, d->bs2, &c.pieces);
  // (the kernels cut the chunk into 64-token parts; score_bs and bs2 above 64 act through the
  // anchors of the kind-2 pieces and, between parts, through the state)
  for (int t = 0; t < 16; ++t) {
    const int ti = t / 4, tj = t % 4;
    c.tile_piece[t] = -1;
    for (int pi = 0; pi < c.pieces.n && ti >= tj; ++pi) {
      const gdn2::Piece& p = c.pieces.p[pi];
      if (16 * ti >= p.row0 && 16 * ti < p.row0 + p.P && 16 * tj >= p.col0 && 16 * tj < p.col0 + p.P)
        c.tile_piece[t] = pi;
    }
  }
  return c;
}

struct Dims {
  size_t n_chunks, n_bh, nc, tD, tT, DD, D;
};
Dims dims(const gdn2_desc* d) {
  Dims x;
  x.nc = (size_t)(d->L / gdn2::T);
  x.n_bh = (size_t)d->B * d->H;
  x.n_chunks = x.n_bh * x.nc;
  x.D = (size_t)d->D;
  x.tD = (size_t)gdn2::T * d->D;
  x.tT = (size_t)gdn2::T * gdn2::T;
  x.DD = (size_t)d->D * d->D;
  return x;
}

void residual_sizes(const gdn2_desc* d, size_t sz[GDN2_RES_COUNT]) {
  const Dims x = dims(d);
  sz[GDN2_RES_AQK] = x.n_chunks * x.tT * 4;
  sz[GDN2_RES_A] = x.n_chunks * x.tT * 4;
  const size_t nck = (size_t)gdn2::CkptBlocks((int)x.nc, eff_ckpt(d), damped_group(d)).nblk;
  sz[GDN2_RES_HPRE] = x.n_bh * nck * x.DD * 4;
  sz[GDN2_RES_VNEW] = x.n_chunks * x.tD * 4;
  sz[GDN2_RES_WP] = x.n_chunks * x.tD * 4;
  sz[GDN2_RES_KG] = x.n_chunks * x.tD * 4;
  sz[GDN2_RES_QG] = x.n_chunks * x.tD * 4;
  sz[GDN2_RES_GL] = x.n_chunks * x.D * 4;
}

void residual_offsets(const gdn2_desc* d, size_t off[GDN2_RES_COUNT], size_t* total) {
  size_t sz[GDN2_RES_COUNT];
  residual_sizes(d, sz);
  size_t o = 0;
  for (int i = 0; i < GDN2_RES_COUNT; ++i) {
    off[i] = o;
    o = align_up(o + sz[i]);
  }
  *total = o;
}

// ---- profiling ------------------------------------------------------------------------
struct ProfRec {
  int kid;
  hipEvent_t a, b;
};
struct Prof {
  bool on = false;
  int cap = 0;
  std::vector<ProfRec> pool;
  int used = 0;
} g_prof;

template <class F>
hipError_t timed(int kid, hipStream_t s, F&& launch) {
  ProfRec* rec = nullptr;
  if (g_prof.on && g_prof.used < g_prof.cap) rec = &g_prof.pool[g_prof.used++];
  if (rec) {
    rec->kid = kid;
    hipEventRecord(rec->a, s);
  }
  hipError_t e = launch();
  if (rec) hipEventRecord(rec->b, s);
  return e;
}

// The anchor buffer of the kind-2 pieces (bs2 > 64): two rows of D floats per 64-token part.
size_t anchor_bytes(const gdn2_desc* d) {
  return d->bs2 > gdn2::T ? align_up((size_t)d->B * d->H * (d->L / gdn2::T) * 2 * d->D * 4) : 0;
}
int hip_fail(hipError_t e, const char* what) {
  return fail(GDN2_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Fills it (anchor_kernel) from the raw gate g into buf; *anc = buf, or null when no piece is of
// kind 2 or the pieces are formed exactly (nothing is launched then).
int fill_anchors(const gdn2_desc* d, const gdn2::Cfg& cfg, const void* g, bool bf16, void* buf, hipStream_t s,
                 const float** anc) {
  *anc = nullptr;
  // (the lean diagonal forms its kind-2 pieces exactly, without anchors)
  if (d->bs2 <= gdn2::T || d->diag == GDN2_DIAG_LEAN) return GDN2_OK;
  gdn2::AnchorArgs aa{g, static_cast<float*>(buf), (int)((size_t)d->B * d->H * (d->L / gdn2::T)), d->bs2 / gdn2::T, cfg};
  const hipError_t e = timed(9, s, [&] { return gdn2::launch_anchors(d->D, aa, s, bf16); });
  if (e != hipSuccess) return hip_fail(e, "anchors launch");
  *anc = aa.anc;
  return GDN2_OK;
}

template <class T>
T* at(void* base, size_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(base) + off);
}

}  // namespace

extern "C" {

int gdn2_abi_version(void) { return GDN2_ABI_VERSION; }

const char* gdn2_last_error(void) { return g_err.c_str(); }

int gdn2_residual_layout(const gdn2_desc* d, size_t offsets[GDN2_RES_COUNT], size_t* total_bytes) {
  const int st = validate_residual(d);
  if (st) return st;
  if (!offsets || !total_bytes) return fail(GDN2_ERR_INVALID, "null output pointer");
  residual_offsets(d, offsets, total_bytes);
  return GDN2_OK;
}

// forward workspace (fragment layouts): [U^T | anchors (bs2 > 64 only)], and without a
// residual also [Kg | Wp | Qg | Aqk | gl] (with a residual those live in it).
size_t gdn2_fwd_workspace_bytes(const gdn2_desc* d, int with_residual) {
  if (with_residual ? validate_residual(d) : validate(d)) return 0;
  const Dims x = dims(d);
  size_t n = align_up(x.n_chunks * x.tD * 4) + anchor_bytes(d);
  if (!with_residual)
    n += 3 * align_up(x.n_chunks * x.tD * 4) + align_up(x.n_chunks * x.tT * 4) + align_up(x.n_chunks * x.D * 4);
  return n;
}

// backward workspace: [dv_new | dh_next | dqg | dwp | dkg | dlast | X | Y | EZ (damped) |
// anchors (bs2 > 64)]
size_t gdn2_bwd_workspace_bytes(const gdn2_desc* d) {
  if (validate_residual(d)) return 0;
  const Dims x = dims(d);
  size_t n = 5 * align_up(x.n_chunks * x.tD * 4) + 2 * align_up(x.n_chunks * x.DD * 4) +
             align_up(x.n_chunks * x.D * 4) + anchor_bytes(d);
  if (damped_group(d) > 1) n += align_up(x.n_chunks * x.DD * 4);     // EZ(j + 1) per 64-token part j
  return n;
}

}  // extern "C"

namespace {
// Forward of one segment; q..g are fp32 or (bf16 = true) bfloat16 bits.  reset: null, or (no
// residual) one byte per (batch, head) and chunk, nonzero = zero state entering that chunk.
int fwd_impl(const gdn2_desc* d, const void* q, const void* k, const void* v, const void* w, const void* b,
             const void* g, bool bf16, const float* h0, float* o, float* h_final, void* residual,
             void* workspace, void* stream, const uint8_t* reset = nullptr) {
  int st = residual ? validate_residual(d) : validate(d);
  if (st) return st;
  if (!q || !k || !v || !w || !b || !g || !o || !h_final || !workspace)
    return fail(GDN2_ERR_INVALID, "null tensor pointer");
  const Dims x = dims(d);
  const gdn2::Cfg cfg = make_cfg(d);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  // operands of the scan and the output kernel, all in fragment layout
  size_t o2 = 0;
  auto take = [&](size_t bytes) { float* p = at<float>(workspace, o2); o2 += align_up(bytes); return p; };
  float* uT = take(x.n_chunks * x.tD * 4);
  void* anc_buf = take(anchor_bytes(d));
  // residuals for the backward -- training only; otherwise Kg / Wp / Qg / Aqk / gl live in the
  // workspace and h_pre and v_new are not stored at all (the scan consumes h_pre and v_new
  // itself).  Wp is kept in the orientation the forward scan contracts over keys and Kg in the
  // one the reverse scan does; each scan turns the other one's blocks around in LDS
  // (gdn2_scan.hip).
  float *A = nullptr, *wp, *kg, *qg, *aqk, *gl, *hpre = nullptr, *vnew = nullptr;
  if (residual) {
    size_t off[GDN2_RES_COUNT], tot;
    residual_offsets(d, off, &tot);
    aqk = at<float>(residual, off[GDN2_RES_AQK]);
    A = at<float>(residual, off[GDN2_RES_A]);
    hpre = at<float>(residual, off[GDN2_RES_HPRE]);
    vnew = at<float>(residual, off[GDN2_RES_VNEW]);
    wp = at<float>(residual, off[GDN2_RES_WP]);
    kg = at<float>(residual, off[GDN2_RES_KG]);
    qg = at<float>(residual, off[GDN2_RES_QG]);
    gl = at<float>(residual, off[GDN2_RES_GL]);
  } else {
    kg = take(x.n_chunks * x.tD * 4);
    wp = take(x.n_chunks * x.tD * 4);
    qg = take(x.n_chunks * x.tD * 4);
    aqk = take(x.n_chunks * x.tT * 4);
    gl = take(x.n_chunks * x.D * 4);
  }

  const float* anc = nullptr;
  st = fill_anchors(d, cfg, g, bf16, anc_buf, s, &anc);
  if (st) return st;
  gdn2::WyFwdArgs wa{};
  wa.q = q; wa.k = k; wa.v = v; wa.w = w; wa.b = b; wa.g = g; wa.anc = anc;
  wa.wp_f = wp; wa.uT_f = uT; wa.kg_f = kg; wa.qg_f = qg;
  wa.aqk_f = aqk; wa.A = A; wa.gl = gl;
  wa.n_chunks = (int)x.n_chunks;
  wa.cfg = cfg;
  hipError_t e = timed(0, s, [&] { return gdn2::launch_wy_fwd(d->D, wa, s, bf16); });
  if (e != hipSuccess) return hip_fail(e, "wy_fwd launch");

  // Without a residual the scan computes the output itself and h_pre / v_new never leave it.
  // Training with state_ckpt = K >= 1 likewise, keeping v_new and the state entering each
  // checkpoint block (gdn2::CkptBlocks; the backward recomputes the others).  Training with state_ckpt = 0 keeps every
  // chunk's h_pre and v_new: the scan carries only the state and the output follows
  // chunk-parallel from them.
  const int ck = eff_ckpt(d);
  const bool fused_out = !residual || ck > 0;
  gdn2::ScanFwdArgs sa{wp, kg, uT, gl, h0, qg, aqk, h_final, fused_out ? o : nullptr, hpre, vnew,
                       (int)x.nc, (int)x.n_bh, ck, cfg, reset};
  e = timed(1, s, [&] { return gdn2::launch_scan_fwd(d->D, sa, s); });
  if (e != hipSuccess) return hip_fail(e, "scan_fwd launch");
  if (!fused_out) {
    gdn2::OutFwdArgs oa{qg, aqk, hpre, vnew, o, (int)x.n_chunks, cfg};
    e = timed(5, s, [&] { return gdn2::launch_out_fwd(d->D, oa, s); });
    if (e != hipSuccess) return hip_fail(e, "out_fwd launch");
  }
  return GDN2_OK;
}
}  // namespace

extern "C" {

int gdn2_fwd(const gdn2_desc* d, const float* q, const float* k, const float* v, const float* w,
             const float* b, const float* g, const float* h0, float* o, float* h_final, void* residual,
             void* workspace, void* stream) {
  return fwd_impl(d, q, k, v, w, b, g, false, h0, o, h_final, residual, workspace, stream);
}

int gdn2_fwd_bf16(const gdn2_desc* d, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                  const uint16_t* w, const uint16_t* b, const uint16_t* g, const float* h0, float* o,
                  float* h_final, void* residual, void* workspace, void* stream) {
  return fwd_impl(d, q, k, v, w, b, g, true, h0, o, h_final, residual, workspace, stream);
}

int gdn2_decode(const gdn2_decode_desc* d, const void* q, const void* k, const void* v, const void* w,
                const void* b, const void* g, const float* a_log, const float* dt_bias, const uint8_t* reset,
                const void* state_in, void* o, void* state_out, void* stream) {
  if (!d) return fail(GDN2_ERR_INVALID, "null descriptor");
  if (d->B < 1 || d->H < 1 || d->n_tok < 1) return fail(GDN2_ERR_INVALID, "non-positive shape");
  if ((int64_t)d->B * d->H > (int64_t(1) << 22)) return fail(GDN2_ERR_UNSUPPORTED, "B*H above 4194304");
  if (d->D != 64 && d->D != 128) return fail(GDN2_ERR_UNSUPPORTED, "D in {64, 128} only");
  if (d->seq_ld < d->n_tok) return fail(GDN2_ERR_INVALID, "seq_ld below n_tok");
  for (int32_t f : {d->in_dtype, d->out_dtype, d->state_dtype, d->fuse_prologue, d->cap})
    if (f != 0 && f != 1) return fail(GDN2_ERR_INVALID, "dtype / flag fields must be 0 or 1");
  if (!q || !k || !v || !w || !b || !g || !o || !state_out) return fail(GDN2_ERR_INVALID, "null tensor pointer");
  if (d->fuse_prologue && (!a_log || !dt_bias)) return fail(GDN2_ERR_INVALID, "fuse_prologue needs a_log and dt_bias");
  gdn2::DecodeArgs a{};
  a.q = q; a.k = k; a.v = v; a.w = w; a.b = b; a.g = g;
  a.a_log = a_log; a.dt_bias = dt_bias; a.reset = reset; a.state_in = state_in;
  a.o = o; a.state_out = state_out;
  a.H = d->H; a.n_tok = d->n_tok; a.seq_ld = d->seq_ld;
  a.in_bf16 = d->in_dtype; a.out_bf16 = d->out_dtype; a.state_bf16 = d->state_dtype;
  a.fuse = d->fuse_prologue; a.cap = d->cap;
  a.scale = (float)d->scale; a.tau = (float)d->stability_tau;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const hipError_t e = timed(8, s, [&] { return gdn2::launch_decode(d->D, a, d->B * d->H, s); });
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  return GDN2_OK;
}

int gdn2_fwd_reset(const gdn2_desc* d, int in_dtype, const void* q, const void* k, const void* v,
                   const void* w, const void* b, const void* g, const float* h0, const uint8_t* chunk_reset,
                   float* o, float* h_final, void* workspace, void* stream) {
  if (in_dtype != 0 && in_dtype != 1) return fail(GDN2_ERR_INVALID, "in_dtype must be 0 (fp32) or 1 (bf16)");
  return fwd_impl(d, q, k, v, w, b, g, in_dtype == 1, h0, o, h_final, nullptr, workspace, stream, chunk_reset);
}

}  // extern "C"

namespace {
// Workspace of the allocation-free forward: a file-scope device array, which the code object
// loader places in every GPU the library is loaded on, at that GPU's own address, for the
// life of the process.  Host code never passes `scratch` itself to a kernel (on the host the
// name is only a stand-in for the symbol); it uses the per-device address that
// hipGetSymbolAddress reports, looked up once per device with that device current.
constexpr size_t kScratchBytes = size_t(64) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;     // per device ordinal; null = not looked up yet

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(GDN2_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GDN2_OK;
}
}  // namespace

extern "C" {

int gdn2_fwd_noalloc(const gdn2_desc* d, const float* q, const float* k, const float* v, const float* w,
                     const float* b, const float* g, const float* h0, float* o, float* h_final, void* stream) {
  const int st = validate(d);
  if (st) return st;
  const size_t need = gdn2_fwd_workspace_bytes(d, 0);
  if (need > kScratchBytes)
    return fail(GDN2_ERR_UNSUPPORTED, "gdn2_fwd_noalloc: this call needs " + std::to_string(need) +
                                          " bytes of workspace, above the library's fixed " +
                                          std::to_string(kScratchBytes) + "-byte device scratch");
  void* ws = nullptr;
  const int sa = scratch_address(&ws);
  if (sa) return sa;
  return fwd_impl(d, q, k, v, w, b, g, false, h0, o, h_final, nullptr, ws, stream);
}

int gdn2_bwd(const gdn2_desc* d, const float* q, const float* k, const float* v, const float* w,
             const float* b, const float* g, const void* residual, const float* d_o, const float* d_hf,
             float* dq, float* dk, float* dv, float* dw, float* db, float* dg, float* dh0, void* workspace,
             void* stream) {
  int st = validate_residual(d);
  if (st) return st;
  if (!q || !k || !v || !w || !b || !g || !residual || !d_o || !d_hf || !dq || !dk || !dv || !dw || !db ||
      !dg || !dh0 || !workspace)
    return fail(GDN2_ERR_INVALID, "null tensor pointer");
  const Dims x = dims(d);
  const gdn2::Cfg cfg = make_cfg(d);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  size_t off[GDN2_RES_COUNT], tot;
  residual_offsets(d, off, &tot);
  void* res = const_cast<void*>(residual);
  const float* aqk = at<float>(res, off[GDN2_RES_AQK]);
  const float* A = at<float>(res, off[GDN2_RES_A]);
  const float* hpre = at<float>(res, off[GDN2_RES_HPRE]);
  const float* vnew = at<float>(res, off[GDN2_RES_VNEW]);
  const float* wp = at<float>(res, off[GDN2_RES_WP]);
  const float* kg = at<float>(res, off[GDN2_RES_KG]);
  const float* qg = at<float>(res, off[GDN2_RES_QG]);
  const float* gl = at<float>(res, off[GDN2_RES_GL]);

  size_t o2 = 0;
  float* dvn = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.tD * 4);
  float* dhn = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.DD * 4);
  float* dqg = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.tD * 4);
  float* dwp = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.tD * 4);
  float* dkg = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.tD * 4);
  float* dlast = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.D * 4);
  float* xo = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.tD * 4);
  float* yo = at<float>(workspace, o2); o2 += align_up(x.n_chunks * x.DD * 4);
  float* ez = nullptr;
  if (damped_group(d) > 1) {
    ez = at<float>(workspace, o2);
    o2 += align_up(x.n_chunks * x.DD * 4);
  }
  const float* anc = nullptr;
  st = fill_anchors(d, cfg, g, false, at<float>(workspace, o2), s, &anc);
  if (st) return st;

  gdn2::BwdPreArgs pa{aqk, qg, d_o, xo, yo, (int)x.n_chunks, cfg};
  hipError_t e = timed(6, s, [&] { return gdn2::launch_bwd_pre(d->D, pa, s); });
  if (e != hipSuccess) return hip_fail(e, "bwd_pre launch");

  gdn2::ScanBwdArgs sa{wp, kg, gl, xo, yo, d_hf, dvn, dhn, dh0, ez, (int)x.nc, (int)x.n_bh, cfg};
  e = timed(2, s, [&] { return gdn2::launch_scan_bwd(d->D, sa, s); });
  if (e != hipSuccess) return hip_fail(e, "scan_bwd launch");

  if (d->state_ckpt > 0) {
    // the states entering the chunks are recomputed from the checkpoints inside the reductions
    gdn2::BwdStateRcArgs ba{d_o, dvn, vnew, hpre, dhn, kg, gl, ez, dqg, dwp, dkg, dlast,
                            (int)x.nc, (int)x.n_bh, eff_ckpt(d), cfg};
    e = timed(7, s, [&] { return gdn2::launch_bwd_state_rc(d->D, ba, s); });
    if (e != hipSuccess) return hip_fail(e, "bwd_state_rc launch");
  } else {
    gdn2::BwdStateArgs ba{d_o, dvn, vnew, hpre, dhn, dqg, dwp, dkg, dlast, (int)x.n_chunks, cfg};
    e = timed(3, s, [&] { return gdn2::launch_bwd_state(d->D, ba, s); });
    if (e != hipSuccess) return hip_fail(e, "bwd_state launch");
  }

  gdn2::BwdWyArgs wa{q, k, v, w, b, g, A, d_o, vnew, dvn, anc, dqg, dwp, dkg, dlast,
                     dq, dk, dv, dw, db, dg, (int)x.n_chunks, cfg};
  e = timed(4, s, [&] { return gdn2::launch_bwd_wy(d->D, wa, s); });
  if (e != hipSuccess) return hip_fail(e, "bwd_wy launch");
  return GDN2_OK;
}

int gdn2_wy_stage(const gdn2_desc* d, const float* q, const float* k, const float* v, const float* w,
                  const float* b, const float* g, float* aqk, float* akk, float* A, float* wp, float* u,
                  float* kg, float* qg, float* gl, void* stream) {
  int st = validate(d);
  if (st) return st;
  if (d->bt != gdn2::T)
    return fail(GDN2_ERR_UNSUPPORTED, "gdn2_wy_stage reports chunks of 64 tokens: use bt == 64");
  if (!q || !k || !v || !w || !b || !g || !aqk || !wp || !u || !kg || !qg || !gl)
    return fail(GDN2_ERR_INVALID, "null tensor pointer");
  const Dims x = dims(d);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  gdn2::WyFwdArgs wa{};
  wa.q = q; wa.k = k; wa.v = v; wa.w = w; wa.b = b; wa.g = g;
  wa.A = A; wa.gl = gl; wa.aqk = aqk; wa.akk = akk; wa.wp = wp; wa.u = u; wa.kg = kg; wa.qg = qg;
  wa.n_chunks = (int)x.n_chunks;
  wa.cfg = make_cfg(d);
  hipError_t e = timed(0, s, [&] { return gdn2::launch_wy_fwd(d->D, wa, s); });
  if (e != hipSuccess) return hip_fail(e, "wy_fwd launch");
  return GDN2_OK;
}

int gdn2_scores(const gdn2_desc* d, const float* q, const float* k, const float* b, const float* gc, float* aqk,
                float* akk, void* stream) {
  int st = validate(d);
  if (st) return st;
  if (d->bt != gdn2::T)
    return fail(GDN2_ERR_UNSUPPORTED, "gdn2_scores reports chunks of 64 tokens: use bt == 64");
  if (!q || !k || !b || !gc || !aqk || !akk) return fail(GDN2_ERR_INVALID, "null tensor pointer");
  const Dims x = dims(d);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  gdn2::WyFwdArgs wa{};
  // v and w are not read (no U is requested); they point at q so that no pointer is null
  wa.q = q; wa.k = k; wa.v = q; wa.w = q; wa.b = b; wa.g = gc;
  wa.g_is_gc = 1;
  wa.aqk = aqk; wa.akk = akk;
  wa.n_chunks = (int)x.n_chunks;
  wa.cfg = make_cfg(d);
  hipError_t e = timed(0, s, [&] { return gdn2::launch_wy_fwd(d->D, wa, s); });
  if (e != hipSuccess) return hip_fail(e, "wy_fwd launch");
  return GDN2_OK;
}

int gdn2_debug_gemm(int mode, const float* A, const float* B, float* C, int M, int N, int K, void* stream) {
  if (mode < 0 || mode > 2) return fail(GDN2_ERR_INVALID, "unknown dot mode");
  if (M <= 0 || N <= 0 || K <= 0 || M > 64 || N > 64 || K > 128 || M % 16 || N % 16 || K % 16)
    return fail(GDN2_ERR_INVALID, "gemm probe shape");
  if (!A || !B || !C) return fail(GDN2_ERR_INVALID, "null tensor pointer");
  hipError_t e = gdn2::launch_gemm_probe(mode, A, B, C, M, N, K, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "gemm probe launch");
  return GDN2_OK;
}

int gdn2_debug_stream(int mode, const void* src, void* dst, size_t bytes, void* stream) {
  if (mode < 0 || mode > 2) return fail(GDN2_ERR_INVALID, "stream probe mode must be 0 (copy), 1 (read) or 2 (fill)");
  if (bytes == 0 || bytes % 4096) return fail(GDN2_ERR_INVALID, "stream probe bytes must be a positive multiple of 4096");
  if (bytes / 4096 > 0x7fffffffu) return fail(GDN2_ERR_INVALID, "stream probe bytes too large");
  if ((mode != 2 && !src) || !dst) return fail(GDN2_ERR_INVALID, "null buffer pointer");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15)
    return fail(GDN2_ERR_INVALID, "stream probe buffers must be 16-byte aligned");
  hipError_t e = gdn2::launch_stream_probe(mode, src, dst, bytes / 16, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "stream probe launch");
  return GDN2_OK;
}

int gdn2_debug_mfma(int blocks, int iters, float* out, void* stream) {
  if (blocks < 1 || blocks > (1 << 20) || iters < 1 || iters > (1 << 20))
    return fail(GDN2_ERR_INVALID, "mfma probe blocks and iters must be in [1, 2^20]");
  if (!out) return fail(GDN2_ERR_INVALID, "null buffer pointer");
  hipError_t e = gdn2::launch_mfma_probe(blocks, iters, out, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "mfma probe launch");
  return GDN2_OK;
}

int gdn2_prof_begin(int max_launches) {
  if (max_launches <= 0) return fail(GDN2_ERR_INVALID, "max_launches must be positive");
  while ((int)g_prof.pool.size() < max_launches) {
    ProfRec r{};
    if (hipEventCreate(&r.a) != hipSuccess || hipEventCreate(&r.b) != hipSuccess)
      return fail(GDN2_ERR_HIP, "hipEventCreate failed");
    g_prof.pool.push_back(r);
  }
  g_prof.cap = max_launches;
  g_prof.used = 0;
  g_prof.on = true;
  return GDN2_OK;
}

int gdn2_prof_end(double ms_sum[GDN2_NUM_KERNELS], int counts[GDN2_NUM_KERNELS]) {
  for (int i = 0; i < GDN2_NUM_KERNELS; ++i) {
    ms_sum[i] = 0.0;
    counts[i] = 0;
  }
  g_prof.on = false;
  for (int i = 0; i < g_prof.used; ++i) {
    ProfRec& r = g_prof.pool[i];
    if (hipEventSynchronize(r.b) != hipSuccess) return fail(GDN2_ERR_HIP, "hipEventSynchronize failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return fail(GDN2_ERR_HIP, "hipEventElapsedTime failed");
    ms_sum[r.kid] += ms;
    counts[r.kid] += 1;
  }
  g_prof.used = 0;
  return GDN2_OK;
}

}  // extern "C"
