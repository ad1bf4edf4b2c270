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
// Products whose contraction runs over the key dimension (Wp h, Kg dh) are computed by waves
// of their own, one token tile each over all keys, with the state read from LDS (every wave
// writes its rows there at the end of a step): no cross-wave reduction.  Products over the
// chunk's time axis (Kg^T v_new, Wp^T dv_new) read v_new / dv_new from LDS in B-operand
// layout.  A-operands stream from global memory as one coalesced
// float4 per lane and block (fragment layout, written by the WY kernel) and are prefetched
// one chunk ahead into the second of two register sets; the chunk loop is unrolled by two so
// the sets never need copying, and all prefetch loads are unconditional so the compiler's
// vmcnt waits stay exact.  Per chunk: two workgroup barriers.
//
// The chain is h -> v_new -> h (dh -> dv_new -> dh).  The forward output o, which needs
// h_pre and v_new but feeds nothing back, is computed inside the forward scan by waves of
// its own (below); the reverse scan's dO terms are computed chunk-parallel before it
// (gdn2_bwd.hip).
//
// Forward (fwd/cd_slim.py:12-30):  v_new = U - Wp h;  h = san(e^gamma h + Kg^T v_new);
//                                  o = san(s Qg h + Aqk v_new)
// Reverse (bwd/mega.py:33-36):     dv_new = san(X + Kg dh);  dh = san(Y + e^gamma dh - Wp^T dv_new)
//                                  with X = Aqk^T dO, Y = Qg^T (s dO)
#include "gdn2_kernels.hpp"

namespace gdn2 {

// Forward scan, with the output fused in when no residual is kept (OUT; in training the
// output waves only carry their state rows).  Eight waves per workgroup (slice of 16 value
// columns of one (batch, head)); per chunk two barriers:
//   window A (after the state h_pre is in LDS):
//     V waves 0-3   v_new tile i = U - Wp[tile i, :] h_pre  (full key contraction, no
//                   cross-wave reduction), written to LDS (and, for the backward, global)
//     O waves 4-7   s Qg[tile j, :] h_pre for their output tile j
//   window B (after v_new is in LDS):
//     every wave w < D/16   h rows of key tile w: h = san(e^gamma h + Kg^T v_new), to LDS
//     O wave j      o tile j = san(s Qg[tile j, :] h_pre + Aqk[tile j, :] v_new)
//                   (fwd/cd_slim.py:24-27)
//   The chain's work (V, state rows) runs at a raised priority and the output's at the
//   default one, so the output takes the MFMA pipe where the chain leaves it idle.
// h_pre in LDS is block kb = key tile in the MFMA result layout of the owning wave, which is
// the B operand of Wp h and the A operand of h^T Qg^T; v_new tiles are in the B-operand
// layout of Kg^T v_new, which is the A operand of v_new^T Aqk^T.  FA(Wp), FA(Qg), FA(Aqk),
// FA(Kg^T), FA(U^T) blocks are loaded as stored (one float4 per lane), one chunk ahead into
// the second of two register sets, interleaved with the MFMAs.
template <int NH>
struct FwdOps {
  float4 x[NH];    // V: FA(Wp) block (i, kb); O: FA(Qg) block (j, kb)
  float4 aq[4];    // O: FA(Aqk) block (j, u), u <= j
  float4 uu;       // V: FA(U^T) block (slice, i)
  float4 kg[4];    // state rows: FA(Kg^T) block (w, u)
  float4 gm;       // state rows: gamma[16w + 4g .. +3]
};

// Prefetch loads for the next chunk are issued in small groups between the MFMA groups of the
// current one (sched_barrier keeps each group where it is written): a wave issuing a burst of
// loads stalls while the CU's vector memory path is busy, and with the loads spread out that
// stall overlaps the MFMAs already in flight.
#define GDN2_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// ROLE < 0: V wave (v_new tile w); ROLE = j >= 0: O wave of output tile j (wave 4 + j).
// OUT = false: no output (the O waves keep only their state rows and the barriers; the
// output is then computed chunk-parallel from h_pre and v_new, gdn2_fwd.hip).
// With Cfg::group = G > 1 (bt = 64 G, wy_eps > 0) the state rows also go to sHd after each part
// j < G - 1 as the damped state h_d(j+1) = state_update(h_d(j), gamma, (1 - eps) Kg^T v_new)
// (h_d(0) = h), from which the V waves compute the next part's v_new (the O waves and the
// state update keep h).
template <int D, int MODE, bool OUT, int ROLE>
__device__ __forceinline__ void scan_fwd_role(const ScanFwdArgs& a, float4* sH, float4* sHd, float4* sV) {
  constexpr int NH = D / 16, NVB = D / 16;
  constexpr bool V = ROLE < 0, O = !V && OUT;
  constexpr int J = V ? 0 : ROLE;
  const float clip = a.cfg.clip, scale = a.cfg.scale;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  const int ti = w & 3;                        // v_new tile of a V wave
  constexpr bool OWNS = V || NH == 8;           // keeps key tile w of the state (w < NH)
  auto base = [&](int c) { return (size_t)bh * nc + (c < nc ? c : nc - 1); };   // clamped chunk

  // A set reset byte zeroes the state entering that chunk.  No load on the sequential path:
  // lane l holds the bytes of chunks 64 m + l of the current block m (fl_cur) and of the next
  // one (fl_nxt), read one block ahead; a step reads its next chunk's byte with readlane.
  const bool has_reset = a.reset != nullptr;
  auto load_flags = [&](int m) -> int {
    const int c = 64 * m + lane_id();
    return (has_reset && c < nc) ? (int)a.reset[(size_t)bh * nc + c] : 0;
  };
  int fl_cur = load_flags(0), fl_nxt = load_flags(1);
  // the byte of chunk c (c >= 1 ascending, one call per step), rotating the blocks as c enters one
  auto reset_at = [&](int c) -> int {
    if (!has_reset || c >= nc) return 0;
    if ((c & 63) == 0) {
      fl_cur = fl_nxt;
      fl_nxt = load_flags(c / 64 + 1);
    }
    return __builtin_amdgcn_readlane(fl_cur, c & 63);
  };
  f4 h = {0.f, 0.f, 0.f, 0.f};
  if (OWNS) {
    if (a.h0 && !(has_reset && __builtin_amdgcn_readlane(fl_cur, 0))) {
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = a.h0[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r];
    }
    sH[w * WAVE + l] = f4_to_float4(h);
  }

  auto load_all = [&](FwdOps<NH>& op, int c) {
    const size_t tb = base(c) * T * D, sb = base(c) * T * T;
    if constexpr (V) {
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) op.x[kb] = ld4(a.wp_f + tb + frag_blk(ti, kb, D) + 4 * l);
      op.uu = ld4(a.uT_f + tb + frag_blk(vb, ti, T) + 4 * l);
    }
    if constexpr (O) {
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) op.x[kb] = ld4(a.qg_f + tb + frag_blk(J, kb, D) + 4 * l);
#pragma unroll
      for (int u = 0; u <= J; ++u) op.aq[u] = ld4(a.aqk_f + sb + frag_blk(J, u, T) + 4 * l);
    }
    if constexpr (OWNS) {
#pragma unroll
      for (int u = 0; u < 4; ++u) op.kg[u] = ld4(a.kgT_f + tb + frag_blk(w, u, T) + 4 * l);
      op.gm = ld4(a.gl + base(c) * D + 16 * w + 4 * g);
    }
  };

  // Cfg::group = G > 1: chunk c is part c % G of a damped big chunk; the state rows keep the
  // damped state h_d of the next part in registers (hdr) and pass it to the V waves through sHd
  const int G = a.cfg.group;
  const float ome = a.cfg.ome;
  f4 hdr = {0.f, 0.f, 0.f, 0.f};
  // checkpoint blocks: the next chunk that starts one and its slot (no division per chunk)
  const CkptBlocks ckb(nc, a.ckpt, G);
  int ck_next = 0, ck_slot = 0;
  // the loop below is unrolled by two from c = 0 (register sets A / B); odd is c's parity
  auto step = [&](const FwdOps<NH>& op, int c, FwdOps<NH>& nx, int cn, auto odd) {
    (void)odd;
    const int part = G > 1 ? c % G : 0;
    const size_t ch = (size_t)bh * nc + c, tb = ch * T * D;
    const size_t tbn = base(cn) * T * D, sbn = base(cn) * T * T;
    const int rst_next = reset_at(cn);
    if (OWNS && a.h_pre_f && c == ck_next) {
      stg4(a.h_pre_f + ((size_t)bh * ckb.nblk + ck_slot) * D * D + frag_blk(vb, w, D) + 4 * l, f4_to_float4(h));
      ck_next += ckb.len(ck_slot);
      ++ck_slot;
    }
    // ---- window A ----
    float4 hb[NH];
    if constexpr (V || O) {
      const float4* src = (V && part > 0) ? sHd : sH;
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) hb[kb] = src[kb * WAVE + l];
    }
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (V) {
      __builtin_amdgcn_s_setprio(2);
      if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
        for (int kb = 0; kb < NH; ++kb) {
          mma16<MODE>(acc, op.x[kb], hb[kb]);
          GDN2_SCHED_FENCE();
          nx.x[kb] = ld4(a.wp_f + tbn + frag_blk(ti, kb, D) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < NH; kb += 2) {
          mma32<MODE>(acc, op.x[kb], hb[kb], op.x[kb + 1], hb[kb + 1]);
          GDN2_SCHED_FENCE();
          nx.x[kb] = ld4(a.wp_f + tbn + frag_blk(ti, kb, D) + 4 * l);
          nx.x[kb + 1] = ld4(a.wp_f + tbn + frag_blk(ti, kb + 1, D) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      }
      drain(acc);
      const float4 vn = sub4(op.uu, f4_to_float4(acc));
      sV[ti * WAVE + l] = vn;
      if (a.v_new_f) stg4(a.v_new_f + tb + frag_blk(vb, ti, T) + 4 * l, vn);
      nx.uu = ld4(a.uT_f + tbn + frag_blk(vb, ti, T) + 4 * l);
    }
    if constexpr (O) {
      // s Qg h_pre needs only h_pre: issued here, at the default priority, so that it fills the
      // MFMA pipe around the V wave's chain (and its LDS / drain latencies) instead of running
      // alone after the state update
      __builtin_amdgcn_s_setprio(0);
      if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
        for (int kb = 0; kb < NH; ++kb) {
          mma16<MODE>(acc, hb[kb], op.x[kb]);
          GDN2_SCHED_FENCE();
          nx.x[kb] = ld4(a.qg_f + tbn + frag_blk(J, kb, D) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < NH; kb += 2) {
          mma32<MODE>(acc, hb[kb], op.x[kb], hb[kb + 1], op.x[kb + 1]);
          GDN2_SCHED_FENCE();
          nx.x[kb] = ld4(a.qg_f + tbn + frag_blk(J, kb, D) + 4 * l);
          nx.x[kb + 1] = ld4(a.qg_f + tbn + frag_blk(J, kb + 1, D) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      }
    }
    __syncthreads();
    // ---- window B ----
    float4 vv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) vv[u] = sV[u * WAVE + l];
    if constexpr (OWNS) {
      __builtin_amdgcn_s_setprio(2);
      // Kg^T v_new: the same chain as the backward's state recompute (gdn2_bwd.hip)
      f4 hn = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          mma16<MODE>(hn, op.kg[u], vv[u]);
          GDN2_SCHED_FENCE();
          nx.kg[u] = ld4(a.kgT_f + tbn + frag_blk(w, u, T) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
          mma32<MODE>(hn, op.kg[u], vv[u], op.kg[u + 1], vv[u + 1]);
          GDN2_SCHED_FENCE();
          nx.kg[u] = ld4(a.kgT_f + tbn + frag_blk(w, u, T) + 4 * l);
          nx.kg[u + 1] = ld4(a.kgT_f + tbn + frag_blk(w, u + 1, T) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      }
      drain(hn);
      const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
      if (part < G - 1) {
        // h_d(part + 1) = san(e^gamma h_d(part) + (1 - eps) Kg^T v_new), h_d(0) = h(0); a reset
        // byte on the next part zeroes it with the state (the rest of the big chunk then starts
        // from zero, damped and true state alike)
        const f4 hb0 = part == 0 ? h : hdr;
#pragma unroll
        for (int e = 0; e < 4; ++e) hdr[e] = rst_next ? 0.f : state_update(hb0[e], gmv[e], ome * hn[e], clip);
        sHd[w * WAVE + l] = f4_to_float4(hdr);   // read in the next step's window A, after its barrier
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = state_update(h[e], gmv[e], hn[e], clip);
      nx.gm = ld4(a.gl + base(cn) * D + 16 * w + 4 * g);
    }
    if constexpr (O) {
      __builtin_amdgcn_s_setprio(0);
      f4 acc2 = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
        for (int u = 0; u <= J; ++u) {
          mma16<MODE>(acc2, vv[u], op.aq[u]);
          GDN2_SCHED_FENCE();
          nx.aq[u] = ld4(a.aqk_f + sbn + frag_blk(J, u, T) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      } else {
#pragma unroll
        for (int u = 0; u <= J; u += 2) {
          if (u + 1 <= J) mma32<MODE>(acc2, vv[u], op.aq[u], vv[u + 1], op.aq[u + 1]);
          else mma16<MODE>(acc2, vv[u], op.aq[u]);
          GDN2_SCHED_FENCE();
          nx.aq[u] = ld4(a.aqk_f + sbn + frag_blk(J, u, T) + 4 * l);
          if (u + 1 <= J) nx.aq[u + 1] = ld4(a.aqk_f + sbn + frag_blk(J, u + 1, T) + 4 * l);
          GDN2_SCHED_FENCE();
        }
      }
      drain(acc, acc2);
      // lane (r, g): o[16 J + r][c0 + 4 g .. + 3]
      stg4(a.o + ((size_t)bh * a.cfg.seq_ld + (size_t)c * T) * D + (size_t)(16 * J + r) * D + c0 + 4 * g,
           make_float4(sanitize(scale * acc[0] + acc2[0], clip), sanitize(scale * acc[1] + acc2[1], clip),
                       sanitize(scale * acc[2] + acc2[2], clip), sanitize(scale * acc[3] + acc2[3], clip)));
    }
    // every wave has read h_pre (window A) before the first barrier, so the new state may
    // overwrite it here
    if (OWNS) {
      if (rst_next) h = f4{0.f, 0.f, 0.f, 0.f};
      sH[w * WAVE + l] = f4_to_float4(h);
    }
    __syncthreads();
  };

  FwdOps<NH> A, B;
  load_all(A, 0);
  __syncthreads();
  int c = 0;
  for (; c + 1 < nc; c += 2) {
    step(A, c, B, c + 1, std::false_type{});
    step(B, c + 1, A, c + 2, std::true_type{});
  }
  if (c < nc) step(A, c, B, c + 1, std::false_type{});
  if (OWNS) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a.hf[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = h[e];
  }
}

template <int D, int MODE, bool OUT>
__global__ __launch_bounds__(8 * WAVE) void scan_fwd_kernel(ScanFwdArgs a) {
  constexpr int NH = D / 16;
  __shared__ float4 sH[NH * WAVE];     // h_pre of the current chunk, [key tile][lane]
  __shared__ float4 sHd[NH * WAVE];    // the damped state of the next part (Cfg::group)
  __shared__ float4 sV[4 * WAVE];      // v_new tiles, [token tile][lane]
  switch (wave_id()) {
    case 4: scan_fwd_role<D, MODE, OUT, 0>(a, sH, sHd, sV); break;
    case 5: scan_fwd_role<D, MODE, OUT, 1>(a, sH, sHd, sV); break;
    case 6: scan_fwd_role<D, MODE, OUT, 2>(a, sH, sHd, sV); break;
    case 7: scan_fwd_role<D, MODE, OUT, 3>(a, sH, sHd, sV); break;
    default: scan_fwd_role<D, MODE, OUT, -1>(a, sH, sHd, sV); break;
  }
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

template <int NH>
struct BwdOps {
  float4 kg[NH];   // dv waves: FA(Kg) block (tp, kb):  Kg[16 tp + r][16 kb + 4 g .. +3]
  float4 wr[NH];   // waves 4-7: FA(Wp) blocks (u, kt), transposed into sWT in window A
  float4 xx;       // dv waves: FA(X^T) block (slice, tp), lane lp: X = Aqk^T dO
  float4 yy;       // FA(Y^T) block (slice, w): Y = s Qg^T dO, this lane's 4 state rows
  float4 gm;       // gamma[16w + 4g .. +3]
};

// Reverse scan, chain only: the dO terms X = Aqk^T dO and Y = s Qg^T dO do not depend on dh and
// come precomputed per chunk (bwd_pre_kernel).  Eight waves; wave w < D/16 keeps key rows
// 16 w .. + 15 of the dh slice in registers.  Per chunk, two barriers:
//   window A  dv waves 0..3 (token tile tp = w): dv_new = san(X + Kg (dh + EZ)) over all D
//             keys, dh read from LDS (sDH, written by every wave at the end of the previous
//             step), the tile to LDS (sDB) and, transposed, to dv_new_f; waves 4..7 (idle
//             otherwise) transpose the chunk's FA(Wp) blocks into sWT = FA(Wp^T) (the residual
//             keeps Wp in the orientation the forward scan contracts over keys);
//   window B  every state wave: z = Wp^T dv_new (its key rows, over the chunk's tokens from
//             sDB, Wp^T from sWT), dh = san(Y + e^gamma dh - z), then dh (+ the next chunk's EZ)
//             to sDH.
// RED: a dv wave (waves 0..3); HELP: a transposing wave (waves 4..7), which also keeps state
// rows when D = 128.  The roles are compile-time parameters, so that each role's code is
// straight-line and its prefetch loads unconditional.
template <int D, int MODE, bool RED, bool HELP>
__device__ __forceinline__ void scan_bwd_role(const ScanBwdArgs& a, float4* sDH, float4* sDB, float* sTr,
                                              float4* sWT, float* sTrs) {
  constexpr int NVB = D / 16, NH = D / 16;
  constexpr bool OWN = RED || NH == 8;     // keeps key tile w of dh
  const float clip = a.cfg.clip;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = lin / NVB, c0 = 16 * vb;
  const int tid = threadIdx.x, l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  const int tp = (tid & 255) >> 6, lp = tid & 63;
  const int J = w & 3;                      // HELP: wave 4 + J

  f4 dh = {0.f, 0.f, 0.f, 0.f};
  if constexpr (OWN) {
#pragma unroll
    for (int e = 0; e < 4; ++e) dh[e] = a.dhf[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r];
    sDH[w * WAVE + l] = f4_to_float4(dh);
  }

  // step s processes chunk nc-1-s; steps past the last are clamped to chunk 0 (loads only)
  auto chunk = [&](int s) { return (size_t)bh * nc + (s < nc ? nc - 1 - s : 0); };
  // wave 4 + J transposes the FA(Wp) blocks m = 0 .. NH - 1 of index J NH + m: key tile
  // (J NH + m) / 4, token tile (J NH + m) % 4
  auto wr_blk = [&](int m) { const int i = J * NH + m; return frag_blk(i % 4, i / 4, D); };
  auto load_all = [&](BwdOps<NH>& op, int s) {
    const size_t ch = chunk(s), tb = ch * T * D;
    if constexpr (RED) {
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) op.kg[kb] = ld4(a.kg_f + tb + frag_blk(tp, kb, D) + 4 * lp);
      op.xx = ld4(a.x_f + tb + frag_blk(vb, tp, T) + 4 * lp);
    }
    if constexpr (HELP) {
#pragma unroll
      for (int m = 0; m < NH; ++m) op.wr[m] = ld4(a.wp_f + tb + wr_blk(m) + 4 * l);
    }
    if constexpr (OWN) {
      op.yy = ld4(a.y_f + ch * D * D + frag_blk(vb, w, D) + 4 * l);
      op.gm = ld4(a.gl + ch * D + 16 * w + 4 * g);
    }
  };

  // Cfg::group = G > 1: chunk c = nc - 1 - s is part c % G of a damped big chunk, and the parts
  // come in reverse.  ez carries EZ(part + 1), the cotangent of the damping correction Delta
  // (gdn2_kernels.hpp, Cfg::group): it is added to dh in this part's Kg dh term (through sDH)
  // and written out for bwd_state_rc, then EZ(part) = eps Wp^T dv_new + e^gamma EZ(part + 1)
  // follows (zero after part 0); the carry dh itself is the undamped form's.
  const int G = a.cfg.group;
  const float eps = a.cfg.wy_eps;
  float4 ez = make_float4(0.f, 0.f, 0.f, 0.f);
  auto carries_ez = [&](int c) { return G > 1 && c >= 0 && c % G < G - 1; };
  auto step = [&](const BwdOps<NH>& op, int s, BwdOps<NH>& nx, int sn, auto sodd) {
    (void)sodd;
    const size_t ch = chunk(s), tb = ch * T * D;
    const size_t chn = chunk(sn), tbn = chn * T * D;
    const int c = nc - 1 - s, part = G > 1 ? c % G : 0;
    const float4 db = f4_to_float4(dh);
    // ---- window A: dv_new tile tp over all keys ----
    if constexpr (RED) {
      float4 hb[NH];
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) hb[kb] = sDH[kb * WAVE + l];
      f4 acc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
        for (int kb = 0; kb < NH; ++kb) {
          mma16<MODE>(acc, op.kg[kb], hb[kb]);
          GDN2_SCHED_FENCE();
          nx.kg[kb] = ld4(a.kg_f + tbn + frag_blk(tp, kb, D) + 4 * lp);
          GDN2_SCHED_FENCE();
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < NH; kb += 2) {
          mma32<MODE>(acc, op.kg[kb], hb[kb], op.kg[kb + 1], hb[kb + 1]);
          GDN2_SCHED_FENCE();
          nx.kg[kb] = ld4(a.kg_f + tbn + frag_blk(tp, kb, D) + 4 * lp);
          nx.kg[kb + 1] = ld4(a.kg_f + tbn + frag_blk(tp, kb + 1, D) + 4 * lp);
          GDN2_SCHED_FENCE();
        }
      }
      drain(acc);
      sDB[tid] = san4(add4(op.xx, f4_to_float4(acc)), clip);
      nx.xx = ld4(a.x_f + tbn + frag_blk(vb, tp, T) + 4 * lp);
    }
    if constexpr (HELP) {
      float4 wt[NH];
      wave_transpose16_n<NH>(sTrs + J * NH * 16 * TRP, op.wr, wt, r, g);
#pragma unroll
      for (int m = 0; m < NH; ++m) sWT[(J * NH + m) * WAVE + l] = wt[m];
      if constexpr (!OWN) {
#pragma unroll
        for (int m = 0; m < NH; ++m) nx.wr[m] = ld4(a.wp_f + tbn + wr_blk(m) + 4 * l);
      }
    }
    float4 dhv = db;
    if constexpr (OWN) {
      // dh entering this chunk's step (mega.py:35) as FA(dh_next) block (w, slice)
      dhv = wave_transpose16(sTr + w * 16 * TRP, db, r, g);
      if (carries_ez(c))
        stg4(a.ez_f + ch * D * D + frag_blk(w, vb, D) + 4 * l, wave_transpose16(sTr + w * 16 * TRP, ez, r, g));
      nx.yy = ld4(a.y_f + chn * D * D + frag_blk(vb, w, D) + 4 * l);
      nx.gm = ld4(a.gl + chn * D + 16 * w + 4 * g);
    }
    __syncthreads();
    // ---- window B: this wave's key rows of dh ----
    if constexpr (OWN) {
      float4 db4[4], wpt[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        db4[u] = sDB[u * WAVE + l];
        wpt[u] = sWT[(4 * w + u) * WAVE + l];
      }
      f4 z = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          mma16<MODE>(z, wpt[u], db4[u]);
          GDN2_SCHED_FENCE();
          if constexpr (HELP) {
#pragma unroll
            for (int m = 2 * u; m < 2 * u + 2; ++m) nx.wr[m] = ld4(a.wp_f + tbn + wr_blk(m) + 4 * l);
          }
          GDN2_SCHED_FENCE();
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
          mma32<MODE>(z, wpt[u], db4[u], wpt[u + 1], db4[u + 1]);
          GDN2_SCHED_FENCE();
          if constexpr (HELP) {
#pragma unroll
            for (int m = 2 * u; m < 2 * u + 4; ++m) nx.wr[m] = ld4(a.wp_f + tbn + wr_blk(m) + 4 * l);
          }
          GDN2_SCHED_FENCE();
        }
      }
      float4 dvv = db;
      if constexpr (RED) dvv = frag_transpose_lds(sDB, tp, lp);     // FA(dv_new) block (tp, slice)
      drain(z);
      const float gmv[4] = {op.gm.x, op.gm.y, op.gm.z, op.gm.w};
      if (G > 1) {
        if (part > 0)
          ez = make_float4(fmaf(exp_nonpos(gmv[0]), ez.x, eps * z[0]), fmaf(exp_nonpos(gmv[1]), ez.y, eps * z[1]),
                           fmaf(exp_nonpos(gmv[2]), ez.z, eps * z[2]), fmaf(exp_nonpos(gmv[3]), ez.w, eps * z[3]));
        else
          ez = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      const float yv[4] = {op.yy.x, op.yy.y, op.yy.z, op.yy.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) dh[e] = sanitize((yv[e] + dh[e] * exp_nonpos(gmv[e])) - z[e], clip);
      // every dv wave has read sDH (window A) before the first barrier: the next chunk's rows
      // may overwrite it here
      const float4 dn = f4_to_float4(dh);
      sDH[w * WAVE + l] = carries_ez(c - 1) ? add4(dn, ez) : dn;
      // stores last: the next step's waits for the prefetch loads above then do not also cover them
      stg4(a.dh_next_f + ch * D * D + frag_blk(w, vb, D) + 4 * l, dhv);
      if constexpr (RED) stg4(a.dv_new_f + tb + frag_blk(tp, vb, D) + 4 * lp, dvv);
    }
    __syncthreads();
  };

  BwdOps<NH> A, B;
  load_all(A, 0);
  __syncthreads();
  int s = 0;
  for (; s + 1 < nc; s += 2) {
    step(A, s, B, s + 1, std::false_type{});
    step(B, s + 1, A, s + 2, std::true_type{});
  }
  if (s < nc) step(A, s, B, s + 1, std::false_type{});
  if constexpr (OWN) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a.dh0[(size_t)bh * D * D + (size_t)(16 * w + 4 * g + e) * D + c0 + r] = dh[e];
  }
}

template <int D, int MODE>
__global__ __launch_bounds__(8 * WAVE) void scan_bwd_kernel(ScanBwdArgs a) {
  constexpr int NH = D / 16;
  __shared__ float4 sDH[NH * WAVE];        // dh (+ EZ) rows of every state wave, B-operand layout, [w][lane]
  __shared__ float4 sDB[4 * WAVE];         // dv_new tiles in B-operand layout, [u][lane]
  __shared__ __attribute__((aligned(16))) float sTr[8 * 16 * TRP];   // per-wave transpose tiles
  __shared__ float4 sWT[NH * 4 * WAVE];    // FA(Wp^T) of the current chunk, [key tile][token tile][lane]
  __shared__ __attribute__((aligned(16))) float sTrs[4 * NH * 16 * TRP];   // transpose tiles of waves 4-7
  if (wave_id() < 4) scan_bwd_role<D, MODE, true, false>(a, sDH, sDB, sTr, sWT, sTrs);
  else scan_bwd_role<D, MODE, false, true>(a, sDH, sDB, sTr, sWT, sTrs);
}

hipError_t launch_scan_fwd(int D, const ScanFwdArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.dot_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (a.o) {
      if (D == 128) hipLaunchKernelGGL((scan_fwd_kernel<128, M, true>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
      else hipLaunchKernelGGL((scan_fwd_kernel<64, M, true>), dim3(a.n_bh * 4), dim3(512), 0, s, a);
    } else {
      if (D == 128) hipLaunchKernelGGL((scan_fwd_kernel<128, M, false>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
      else hipLaunchKernelGGL((scan_fwd_kernel<64, M, false>), dim3(a.n_bh * 4), dim3(512), 0, s, a);
    }
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_scan_bwd(int D, const ScanBwdArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((scan_bwd_kernel<128, M>), dim3(a.n_bh * 8), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((scan_bwd_kernel<64, M>), dim3(a.n_bh * 4), dim3(512), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

}  // namespace gdn2
