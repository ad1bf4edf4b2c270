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
// vmcnt waits stay exact.  Per chunk: two syncs of the waves on the chain (workgroup barriers
// in the reverse scan; in the forward scan, whose output waves trail the chain, LDS counters).
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

// Forward scan, one workgroup per (batch, head, slice of 16 value columns), eight waves:
//   chain waves 0..3  the recurrence.  Wave w computes v_new tile w = U - Wp[tile w, :] h_pre
//                     (window A, full key contraction) and keeps the state rows of key tiles
//                     kt(w, j) = w + 4 j (j < D/64) in registers, updated in window B:
//                     h = san(e^gamma h + Kg^T v_new) (fwd/cd_slim.py:24-27).  Two syncs per
//                     chunk among these four waves only (an LDS counter, below): after window A
//                     (v_new complete in LDS) and after window B (the next h_pre complete).
//   output waves 4..7 (OUT) o tile j = san(s Qg[tile j, :] h_pre + Aqk[tile j, :] v_new)
//                     (fwd/cd_slim.py:25,28), trailing the chain: a chunk's h_pre and v_new are
//                     read as soon as its window-A sync has passed, and the MFMAs run after the
//                     reads are released, at the default priority, in whatever gaps the chain
//                     leaves in the MFMA pipe (the chain waves run at a raised one).
// h_pre and v_new are double-buffered in LDS by chunk parity; the chain writes a buffer only
// after every output wave has released the chunk that used it before (each output wave counts
// its releases on a counter of its own, and the chain checks all four).  All waits are bounded
// spins (a wave that runs out of spins stops waiting and finishes, so the grid always drains;
// the results are then wrong, which no in-range input can cause).  Syncs are LDS counters
// with release increments and acquire loads (workgroup scope): every LDS write before a
// release is visible to a wave whose acquire load sees the increment.
// h_pre in LDS is block kb = key tile in the MFMA result layout of the owning wave, which is
// the B operand of Wp h and the A operand of h^T Qg^T; v_new tiles are in the B-operand
// layout of Kg^T v_new, which is the A operand of v_new^T Aqk^T.  FA(Wp), FA(Qg), FA(Aqk),
// FA(Kg), FA(U^T) blocks are loaded as stored (one float4 per lane), one chunk ahead into
// the second of two register sets, interleaved with the MFMAs; the FA(Kg) blocks are turned
// into FA(Kg^T) blocks by the chain wave itself, between the MFMAs of window A.
template <int NH>
struct ChainOps {
  float4 x[NH];            // FA(Wp) block (w, kb)
  float4 uu;               // FA(U^T) block (slice, w)
  float4 kg[NH / 4][4];    // FA(Kg) blocks (u, kt(w, j)), turned into FA(Kg^T) blocks (kt, u) in window A
  float4 gm[NH / 4];       // gamma of key tile kt(w, j)
};
template <int NH>
struct OutOps {
  float4 x[NH];            // FA(Qg) block (j, kb)
  float4 aq[4];            // FA(Aqk) block (j, u), u <= j
};

// Prefetch loads for the next chunk are issued in small groups between the MFMA groups of the
// current one (sched_barrier keeps each group where it is written): a wave issuing a burst of
// loads stalls while the CU's vector memory path is busy, and with the loads spread out that
// stall overlaps the MFMAs already in flight.
#define GDN2_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// Workgroup-local syncs on monotonic LDS counters.
constexpr int SCAN_SPIN_MAX = 1 << 22;
// One increment per wave: lane 0 alone issues the add (an add from every active lane would
// count the wave's active lanes).
__device__ __forceinline__ void lds_release_add(unsigned* ctr) {
  if (lane_id() == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Waits until *ctr >= target; ok turns false (and stays false, so later waits return at once)
// when the spin budget runs out.  SLEEP: pause between polls (the output waves, which wait
// long and should leave the issue slots to the chain); the chain waves poll back to back.
template <bool SLEEP>
__device__ __forceinline__ void lds_acquire_wait(unsigned* ctr, unsigned target, bool& ok) {
  if (!ok) return;
  for (int i = 0; i < SCAN_SPIN_MAX; ++i) {
    if (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
    if constexpr (SLEEP) __builtin_amdgcn_s_sleep(1);
  }
  ok = false;
}
// Waits until each of the counters ctr[0 .. N-1] is >= target.  seen is the smallest value of
// this wave's last read: when it already satisfies the target the sync has happened and
// nothing is read.  Waves that are not in lockstep with one another (the output waves) release a
// counter each: with one shared counter the increments of a wave that is ahead could stand in
// for those of a wave that is behind.  (The chain waves share one counter: none of them passes
// a sync point before all of them have released it, so its sum is exact.)  The N counters are
// read with relaxed loads in one round trip, then an acquire fence on LDS orders what follows.
template <int N>
__device__ __forceinline__ void lds_acquire_wait_each(unsigned* ctr, unsigned target, unsigned& seen, bool& ok) {
  if (!ok || seen >= target) return;
  for (int i = 0; i < SCAN_SPIN_MAX; ++i) {
    unsigned m = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < N; ++j) m = min(m, __hip_atomic_load(ctr + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    seen = m;
    if (m >= target) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
      return;
    }
  }
  ok = false;
}

struct ScanFwdShared {
  unsigned cbar;           // chain syncs, 4 per sync point: k = 0 after the initial state is in
                           // LDS, k = 2 c + 1 after chunk c's window A, k = 2 c + 2 after its B
  unsigned odone[4];       // output wave J's releases: 1 per chunk
};
// cbar once sync point k has passed
__device__ __forceinline__ unsigned cbar_at(int k) { return 4u * (unsigned)(k + 1); }

// Chain wave w.  With Cfg::group = G > 1 (bt = 64 G, wy_eps > 0) the state rows also go to sHd
// after each part j < G - 1 as the damped state h_d(j+1) = state_update(h_d(j), gamma,
// (1 - eps) Kg^T v_new) (h_d(0) = h), from which the next part's v_new is computed (the output
// and the state update keep h).
template <int D, int MODE, bool OUT>
__device__ __forceinline__ void scan_fwd_chain(const ScanFwdArgs& a, ScanFwdShared* sh, float4* sH, float4* sHd,
                                               float4* sV, float* sTrK) {
  constexpr int NH = D / 16, NVB = D / 16, NJ = NH / 4;
  const float clip = a.cfg.clip;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  // (batch, head)s in reverse order: the WY build writes them in ascending order, so the first
  // workgroups read the lines written last, the likeliest to be still cached (when the grid
  // takes several rounds, config 4: about -1 % of the scan; config 2: -0.9 us)
  const int vb = lin % NVB, bh = a.n_bh - 1 - lin / NVB, c0 = 16 * vb;
  const int l = lane_id(), r = l & 15, g = l >> 4, w = wave_id();
  auto kt = [&](int j) { return w + 4 * j; };
  auto base = [&](int c) { return (size_t)bh * nc + (c < nc ? c : nc - 1); };   // clamped chunk
  bool ok = true;
  unsigned odone_seen = 0;      // the output waves trail by about a chunk: one read serves several waits

  // A set reset byte zeroes the state entering that chunk.  No load on the sequential path:
  // lane l holds the bytes of chunks 64 m + l of the current block m (fl_cur) and of the next
  // one (fl_nxt), read one block ahead; a step reads its next chunk's byte with readlane.
  const bool has_reset = a.reset != nullptr;
  auto load_flags = [&](int m) -> int {
    const int c = 64 * m + lane_id();
    return (has_reset && c < nc) ? (int)a.reset[(size_t)bh * nc + c] : 0;
  };
  int fl_cur = load_flags(0), fl_nxt = load_flags(1);
  auto reset_at = [&](int c) -> int {
    if (!has_reset || c >= nc) return 0;
    if ((c & 63) == 0) {
      fl_cur = fl_nxt;
      fl_nxt = load_flags(c / 64 + 1);
    }
    return __builtin_amdgcn_readlane(fl_cur, c & 63);
  };
  f4 h[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    h[j] = f4{0.f, 0.f, 0.f, 0.f};
    if (a.h0 && !(has_reset && __builtin_amdgcn_readlane(fl_cur, 0))) {
#pragma unroll
      for (int e = 0; e < 4; ++e) h[j][e] = a.h0[(size_t)bh * D * D + (size_t)(16 * kt(j) + 4 * g + e) * D + c0 + r];
    }
    sH[kt(j) * WAVE + l] = f4_to_float4(h[j]);     // buffer 0: h_pre of chunk 0
  }
  // sync point 0: every chain wave reads every key tile of chunk 0's h_pre
  lds_release_add(&sh->cbar);
  lds_acquire_wait<false>(&sh->cbar, cbar_at(0), ok);

  auto load_all = [&](ChainOps<NH>& op, int c) {
    const size_t tb = base(c) * T * D;
#pragma unroll
    for (int kb = 0; kb < NH; ++kb) op.x[kb] = ld4(a.wp_f + tb + frag_blk(w, kb, D) + 4 * l);
    op.uu = ld4(a.uT_f + tb + frag_blk(vb, w, T) + 4 * l);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int u = 0; u < 4; ++u) op.kg[j][u] = ld4(a.kg_f + tb + frag_blk(u, kt(j), D) + 4 * l);
      op.gm[j] = ld4(a.gl + base(c) * D + 16 * kt(j) + 4 * g);
    }
  };

  const int G = a.cfg.group;
  const float ome = a.cfg.ome;
  f4 hdr[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) hdr[j] = f4{0.f, 0.f, 0.f, 0.f};
  // checkpoint blocks: the next chunk that starts one and its slot (no division per chunk)
  const CkptBlocks ckb(nc, a.ckpt, G);
  int ck_next = 0, ck_slot = 0;
  __builtin_amdgcn_s_setprio(2);
  auto step = [&](const ChainOps<NH>& op, int c, ChainOps<NH>& nx, int cn, auto odd) {
    constexpr int buf = decltype(odd)::value ? 1 : 0;      // c & 1
    const int part = G > 1 ? c % G : 0;
    const size_t ch = (size_t)bh * nc + c, tb = ch * T * D;
    const size_t tbn = base(cn) * T * D;
    const int rst_next = reset_at(cn);
    float4* sHc = sH + buf * NH * WAVE;            // h_pre of this chunk
    float4* sHn = sH + (1 - buf) * NH * WAVE;      // h_pre of the next one
    float4* sVc = sV + buf * 4 * WAVE;
    if (a.h_pre_f && c == ck_next) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        stg4(a.h_pre_f + ((size_t)bh * ckb.nblk + ck_slot) * D * D + frag_blk(vb, kt(j), D) + 4 * l, f4_to_float4(h[j]));
      ck_next += ckb.len(ck_slot);
      ++ck_slot;
    }
    // ---- window A: v_new tile w ----
    float4 hb[NH];
    {
      const float4* src = part > 0 ? sHd : sHc;
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) hb[kb] = src[kb * WAVE + l];
    }
    // window B's A operands, FA(Kg^T) blocks (kt(w, j), u): this chunk's FA(Kg) blocks (u, kt)
    // turned around through the wave's transpose tile, one per MFMA group while the chain runs
    // (the residual keeps Kg in the orientation the reverse scan contracts over keys)
    float4 kgt[NJ][4];
    static_assert(4 * NJ == NH, "one transpose per key block of the chain");
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) {
        mma16<MODE>(acc, op.x[kb], hb[kb]);
        GDN2_SCHED_FENCE();
        nx.x[kb] = ld4(a.wp_f + tbn + frag_blk(w, kb, D) + 4 * l);
        kgt[kb / 4][kb % 4] = wave_transpose16(sTrK, op.kg[kb / 4][kb % 4], r, g);
        GDN2_SCHED_FENCE();
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < NH; kb += 2) {
        mma32<MODE>(acc, op.x[kb], hb[kb], op.x[kb + 1], hb[kb + 1]);
        GDN2_SCHED_FENCE();
        nx.x[kb] = ld4(a.wp_f + tbn + frag_blk(w, kb, D) + 4 * l);
        nx.x[kb + 1] = ld4(a.wp_f + tbn + frag_blk(w, kb + 1, D) + 4 * l);
        kgt[kb / 4][kb % 4] = wave_transpose16(sTrK, op.kg[kb / 4][kb % 4], r, g);
        kgt[kb / 4][kb % 4 + 1] = wave_transpose16(sTrK, op.kg[kb / 4][kb % 4 + 1], r, g);
        GDN2_SCHED_FENCE();
      }
    }
    drain(acc);
    const float4 vn = sub4(op.uu, f4_to_float4(acc));
    // the output waves have released chunk c - 2, which used this v_new buffer
    if constexpr (OUT) lds_acquire_wait_each<4>(sh->odone, (unsigned)(c > 1 ? c - 1 : 0), odone_seen, ok);
    sVc[w * WAVE + l] = vn;
    if (a.v_new_f) stg4(a.v_new_f + tb + frag_blk(vb, w, T) + 4 * l, vn);
    nx.uu = ld4(a.uT_f + tbn + frag_blk(vb, w, T) + 4 * l);
    lds_release_add(&sh->cbar);
    lds_acquire_wait<false>(&sh->cbar, cbar_at(2 * c + 1), ok);
    // ---- window B: the state rows of key tiles kt(w, j) ----
    float4 vv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) vv[u] = sVc[u * WAVE + l];
    f4 hn[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) hn[j] = f4{0.f, 0.f, 0.f, 0.f};
    // Kg^T v_new: the same chain per key tile as the backward's state recompute (gdn2_bwd.hip);
    // the key tiles' chains interleaved
    if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) mma16<MODE>(hn[j], kgt[j][u], vv[u]);
        GDN2_SCHED_FENCE();
#pragma unroll
        for (int j = 0; j < NJ; ++j) nx.kg[j][u] = ld4(a.kg_f + tbn + frag_blk(u, kt(j), D) + 4 * l);
        GDN2_SCHED_FENCE();
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; u += 2) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) mma32<MODE>(hn[j], kgt[j][u], vv[u], kgt[j][u + 1], vv[u + 1]);
        GDN2_SCHED_FENCE();
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          nx.kg[j][u] = ld4(a.kg_f + tbn + frag_blk(u, kt(j), D) + 4 * l);
          nx.kg[j][u + 1] = ld4(a.kg_f + tbn + frag_blk(u + 1, kt(j), D) + 4 * l);
        }
        GDN2_SCHED_FENCE();
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) drain(hn[j]);
    // the output waves have released chunk c - 1, whose h_pre buffer the next h_pre overwrites
    if constexpr (OUT) lds_acquire_wait_each<4>(sh->odone, (unsigned)c, odone_seen, ok);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float gmv[4] = {op.gm[j].x, op.gm[j].y, op.gm[j].z, op.gm[j].w};
      if (part < G - 1) {
        // h_d(part + 1) = san(e^gamma h_d(part) + (1 - eps) Kg^T v_new), h_d(0) = h(0); a reset
        // byte on the next part zeroes it with the state (the rest of the big chunk then starts
        // from zero, damped and true state alike)
        const f4 hb0 = part == 0 ? h[j] : hdr[j];
#pragma unroll
        for (int e = 0; e < 4; ++e) hdr[j][e] = rst_next ? 0.f : state_update(hb0[e], gmv[e], ome * hn[j][e], clip);
        sHd[kt(j) * WAVE + l] = f4_to_float4(hdr[j]);   // read in the next step's window A, after its sync
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) h[j][e] = state_update(h[j][e], gmv[e], hn[j][e], clip);
      nx.gm[j] = ld4(a.gl + base(cn) * D + 16 * kt(j) + 4 * g);
      if (rst_next) h[j] = f4{0.f, 0.f, 0.f, 0.f};
      sHn[kt(j) * WAVE + l] = f4_to_float4(h[j]);
    }
    lds_release_add(&sh->cbar);
    lds_acquire_wait<false>(&sh->cbar, cbar_at(2 * c + 2), ok);
  };

  ChainOps<NH> A, B;
  load_all(A, 0);
  int c = 0;
  for (; c + 1 < nc; c += 2) {
    step(A, c, B, c + 1, std::false_type{});
    step(B, c + 1, A, c + 2, std::true_type{});
  }
  if (c < nc) step(A, c, B, c + 1, std::false_type{});
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) a.hf[(size_t)bh * D * D + (size_t)(16 * kt(j) + 4 * g + e) * D + c0 + r] = h[j][e];
}

// Output wave J (wave 4 + J).  J is a compile-time parameter: the causal Aqk v_new chain's
// length depends on it, and a runtime branch between the MFMAs of a chain would let the
// compiler copy the accumulator at the merge point, right after an (opaque) asm MFMA.
template <int D, int MODE, int J>
__device__ __forceinline__ void scan_fwd_out(const ScanFwdArgs& a, ScanFwdShared* sh, const float4* sH,
                                             const float4* sV) {
  constexpr int NH = D / 16, NVB = D / 16;
  const float clip = a.cfg.clip, scale = a.cfg.scale;
  const int nc = a.nc;
  const int lin = xcd_remap(gridDim.x);
  const int vb = lin % NVB, bh = a.n_bh - 1 - lin / NVB, c0 = 16 * vb;   // as the chain waves
  const int l = lane_id(), r = l & 15, g = l >> 4;
  auto base = [&](int c) { return (size_t)bh * nc + (c < nc ? c : nc - 1); };
  bool ok = true;
  auto load_all = [&](OutOps<NH>& op, int c) {
    const size_t tb = base(c) * T * D, sb = base(c) * T * T;
#pragma unroll
    for (int kb = 0; kb < NH; ++kb) op.x[kb] = ld4(a.qg_f + tb + frag_blk(J, kb, D) + 4 * l);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (u <= J) op.aq[u] = ld4(a.aqk_f + sb + frag_blk(J, u, T) + 4 * l);
  };
  auto step = [&](const OutOps<NH>& op, int c, OutOps<NH>& nx, int cn, auto odd) {
    constexpr int buf = decltype(odd)::value ? 1 : 0;
    const size_t tbn = base(cn) * T * D, sbn = base(cn) * T * T;
    // this chunk's h_pre and v_new are complete once its window-A sync has passed
    lds_acquire_wait<true>(&sh->cbar, cbar_at(2 * c + 1), ok);
    float4 hb[NH], vv[4];
#pragma unroll
    for (int kb = 0; kb < NH; ++kb) hb[kb] = sH[buf * NH * WAVE + kb * WAVE + l];
#pragma unroll
    for (int u = 0; u < 4; ++u) vv[u] = u <= J ? sV[buf * 4 * WAVE + u * WAVE + l] : make_float4(0.f, 0.f, 0.f, 0.f);
    lds_release_add(&sh->odone[J]);    // the release waits for the reads above
    f4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE == DOT_HIGHEST) {
#pragma unroll
      for (int kb = 0; kb < NH; ++kb) {
        mma16<MODE>(acc, hb[kb], op.x[kb]);
        GDN2_SCHED_FENCE();
        nx.x[kb] = ld4(a.qg_f + tbn + frag_blk(J, kb, D) + 4 * l);
        GDN2_SCHED_FENCE();
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u > J) continue;
        mma16<MODE>(acc2, vv[u], op.aq[u]);
        GDN2_SCHED_FENCE();
        nx.aq[u] = ld4(a.aqk_f + sbn + frag_blk(J, u, T) + 4 * l);
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
#pragma unroll
      for (int u = 0; u < 4; u += 2) {
        if (u > J) continue;
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
    stg4_keep(a.o + ((size_t)bh * a.cfg.seq_ld + (size_t)c * T) * D + (size_t)(16 * J + r) * D + c0 + 4 * g,
         make_float4(sanitize(scale * acc[0] + acc2[0], clip), sanitize(scale * acc[1] + acc2[1], clip),
                     sanitize(scale * acc[2] + acc2[2], clip), sanitize(scale * acc[3] + acc2[3], clip)));
  };
  OutOps<NH> A, B;
  load_all(A, 0);
  int c = 0;
  for (; c + 1 < nc; c += 2) {
    step(A, c, B, c + 1, std::false_type{});
    step(B, c + 1, A, c + 2, std::true_type{});
  }
  if (c < nc) step(A, c, B, c + 1, std::false_type{});
}

template <int D, int MODE, bool OUT>
__global__ __launch_bounds__(8 * WAVE) void scan_fwd_kernel(ScanFwdArgs a) {
  constexpr int NH = D / 16;
  __shared__ float4 sH[2 * NH * WAVE];     // h_pre by chunk parity, [buffer][key tile][lane]
  __shared__ float4 sHd[NH * WAVE];        // the damped state of the next part (Cfg::group)
  __shared__ float4 sV[2 * 4 * WAVE];      // v_new tiles by chunk parity, [buffer][token tile][lane]
  __shared__ __attribute__((aligned(16))) float sTrK[4 * 16 * TRP];   // chain waves' transpose tiles
  __shared__ ScanFwdShared sh;
  if (threadIdx.x == 0) {
    sh.cbar = 0;
    sh.odone[0] = sh.odone[1] = sh.odone[2] = sh.odone[3] = 0;
  }
  __syncthreads();
  if constexpr (OUT) {
    switch (wave_id()) {
      case 4: scan_fwd_out<D, MODE, 0>(a, &sh, sH, sV); break;
      case 5: scan_fwd_out<D, MODE, 1>(a, &sh, sH, sV); break;
      case 6: scan_fwd_out<D, MODE, 2>(a, &sh, sH, sV); break;
      case 7: scan_fwd_out<D, MODE, 3>(a, &sh, sH, sV); break;
      default: scan_fwd_chain<D, MODE, OUT>(a, &sh, sH, sHd, sV, sTrK + wave_id() * 16 * TRP); break;
    }
  } else {
    if (wave_id() < 4) scan_fwd_chain<D, MODE, OUT>(a, &sh, sH, sHd, sV, sTrK + wave_id() * 16 * TRP);
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
