// Backward kernels of the GDN-2 operator on gfx950 (the reference fuses all of this into
// one reverse loop per (batch, head), bwd/mega.py:9-58; here the sequential part and the
// chunk-parallel part are separate launches so that the chunk-parallel part fills the GPU).
//
//   bwd_pre_kernel   one workgroup per chunk: the reverse scan's dO terms Aqk^T dO and
//                    Qg^T (s dO), which do not depend on the carried state     (mega.py:34-35)
//   (the reverse state scan, dv_new and dh_next per chunk, is in gdn2_scan.hip)
//   bwd_state_kernel one workgroup per chunk: the reductions over the value dimension
//                      dQg = (s dO) h_pre^T, dWp = -dv_new h_pre^T, dKg = v_new dh_next^T
//                    (written as FA(dQg^T), FA(dWp^T), FA(dKg^T)) and the row sums
//                    sum_v dh_next * h_pre                                    (mega.py:38-40,50)
//   bwd_wy_kernel    one workgroup per chunk: dAqk, dA, dkb, dwv, the WY-inverse backward
//                    dAkk = -(1-eps) strict(A^T (dA A^T)), the elementwise gate gradients,
//                    B4 (VJP of the two-level scores) and B5 (reverse cumsum)
//                                                     (mega.py:32-59, bwd/b4.py:45-97)
#include "gdn2_kernels.hpp"

namespace gdn2 {

// ------------------------------------------------------------------------------------
// bwd_state: one workgroup per chunk, D/16 waves.  Wave w owns key tile w (key rows
// 16 w .. 16 w + 15) of the three outputs and accumulates, over the value blocks kb,
//   dQg^T tile (w, ti) += h_pre[w-rows, kb] . (s dO)[ti-rows, kb]^T
//   dWp^T tile (w, ti) += h_pre[w-rows, kb] . (-dv_new)[ti-rows, kb]^T
//   dKg^T tile (w, ti) += dh_next[w-rows, kb] . v_new[ti-rows, kb]^T
// The MFMA operands must be value-contiguous per lane.  The A operands of one kb (the 64 x 16
// slabs of s dO, -dv_new and v_new, 12 KB), which every wave needs, are staged once per
// workgroup in LDS in operand order (double-buffered, one barrier per kb); v_new arrives as
// FA(v_new^T), whose blocks are the needed blocks in the MFMA result layout, and is
// transposed while it is written to LDS.  The B operands are per wave: dh_next (FA, from the
// reverse scan) straight from global memory, h_pre (FA(h_pre^T) from the forward scan)
// through a per-wave LDS transpose.  Two or more workgroups share a CU, so one's barrier
// waits and loads overlap the others' MFMAs.  The accumulator of tile (ti, w) is block
// (w, ti) of FA(out^T): one float4 store.
// ------------------------------------------------------------------------------------
template <int D, int B3>
__global__ __launch_bounds__(D / 16 * WAVE) __attribute__((amdgpu_waves_per_eu(D == 128 ? 4 : 1))) void bwd_state_kernel(BwdStateArgs a) {
  constexpr int NKB = D / 16, NW = D / 16, NT = NW * WAVE, SLAB = 12 * WAVE;   // float4 per slab
  constexpr int NST = (SLAB + NT - 1) / NT;                                      // staged per thread
  __shared__ float4 sA[2 * SLAB];                   // [buf][mat * 4 + ti][lane]
  __shared__ __attribute__((aligned(16))) float sTr[NW * 16 * TRP];
  const Cfg& cf = a.cfg;
  const int chunk = blockIdx.x, tid = threadIdx.x, kt = wave_id(), l = lane_id(), r = l & 15, g = l >> 4;
  const size_t tb = (size_t)chunk * T * D, hb = (size_t)chunk * D * D, tio = io_off<D>(cf, chunk);
  const float sc = cf.scale;
  float* tr = sTr + kt * 16 * TRP;

  // staging item f of a slab: mat = f / 256 (0: s dO, 1: -dv_new, 2: v_new), ti = f / 64 % 4,
  // lane f % 64 of the operand block (ti, kb).  Slabs and B operands are fetched two value
  // blocks ahead (register sets by kb parity; the kb loop is unrolled by two so that every
  // index is static): one block's 48 MFMAs per wave are too short to cover a load.
  float4 st[2][NST];
  auto fetch = [&](int kb, float4 (&dst)[NST]) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int f = tid + j * NT;
      if (f < SLAB) {
        const int mat = f >> 8, ti = (f >> 6) & 3, ln = f & 63;
        if (mat == 0)
          dst[j] = ld4(a.dout + tio + (16 * ti + (ln & 15)) * D + 16 * kb + 4 * (ln >> 4));
        else if (mat == 1)
          dst[j] = ld4(a.dv_new_f + tb + frag_blk(ti, kb, D) + 4 * ln);
        else
          dst[j] = ld4(a.v_new_f + tb + frag_blk(kb, ti, T) + 4 * ln);
      }
    }
  };
  auto put = [&](int buf, const float4 (&src)[NST]) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int f = tid + j * NT;
      if (f < SLAB) {
        const int mat = f >> 8, ti = (f >> 6) & 3, ln = f & 63;
        float4* dst = sA + buf * SLAB + (mat * 4 + ti) * WAVE;
        if (mat == 0) {
          dst[ln] = scale4(src[j], sc);
        } else if (mat == 1) {
          dst[ln] = scale4(src[j], -1.f);
        } else {
          // lane ln = (rr, gg) holds v_new[16 ti + 4 gg + e][16 kb + rr]: operand lane
          // (4 gg + e) + 16 (rr / 4), component rr % 4
          float* df = reinterpret_cast<float*>(dst);
          const int rr = ln & 15, gg = ln >> 4, base = 4 * (4 * gg + 16 * (rr >> 2)) + (rr & 3);
          df[base] = src[j].x;
          df[base + 4] = src[j].y;
          df[base + 8] = src[j].z;
          df[base + 12] = src[j].w;
        }
      }
    }
  };

  f4 acc[3][4];
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) acc[m][ti] = f4{0.f, 0.f, 0.f, 0.f};
  float part = 0.f;
  float4 hpT[2], dh[2];
  fetch(0, st[0]);
  hpT[0] = ld4(a.h_pre_f + hb + frag_blk(0, kt, D) + 4 * l);
  dh[0] = ld4(a.dh_next_f + hb + frag_blk(kt, 0, D) + 4 * l);
  fetch(1, st[1]);
  hpT[1] = ld4(a.h_pre_f + hb + frag_blk(1, kt, D) + 4 * l);
  dh[1] = ld4(a.dh_next_f + hb + frag_blk(kt, 1, D) + 4 * l);
  put(0, st[0]);
  __syncthreads();
#pragma unroll 2
  for (int kb = 0; kb < NKB; ++kb) {
    const int pb = kb & 1;
    // h_pre block (kt, kb) from FA(h_pre^T) block (kb, kt), its MFMA result layout
    const float4 hp = wave_transpose16(tr, hpT[pb], r, g);
    const float4 dhc = dh[pb];
    if (kb + 2 < NKB) {
      fetch(kb + 2, st[pb]);
      hpT[pb] = ld4(a.h_pre_f + hb + frag_blk(kb + 2, kt, D) + 4 * l);
      dh[pb] = ld4(a.dh_next_f + hb + frag_blk(kt, kb + 2, D) + 4 * l);
    }
    const float4* cur = sA + pb * SLAB;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      mma16<B3>(acc[0][ti], cur[ti * WAVE + l], hp);
      mma16<B3>(acc[1][ti], cur[(4 + ti) * WAVE + l], hp);
      mma16<B3>(acc[2][ti], cur[(8 + ti) * WAVE + l], dhc);
    }
    // sum_v dh_next * h_pre over this lane's 4 values of key row 16 kt + r
    part = fmaf(dhc.x, hp.x, part);
    part = fmaf(dhc.y, hp.y, part);
    part = fmaf(dhc.z, hp.z, part);
    part = fmaf(dhc.w, hp.w, part);
    if (kb + 1 < NKB) put(pb ^ 1, st[pb ^ 1]);
    __syncthreads();
  }
  drain(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
  drain(acc[1][0], acc[1][1], acc[1][2], acc[1][3]);
  drain(acc[2][0], acc[2][1], acc[2][2], acc[2][3]);
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
    const size_t o = tb + frag_blk(kt, ti, T) + 4 * l;
    stg4(a.dqg + o, f4_to_float4(acc[0][ti]));
    stg4(a.dwp + o, f4_to_float4(acc[1][ti]));
    stg4(a.dkg + o, f4_to_float4(acc[2][ti]));
  }
  // the four lanes of key row 16 kt + r hold the value blocks 4 g .. 4 g + 3 of every kb
  part += __shfl_xor(part, 16);
  part += __shfl_xor(part, 32);
  if (g == 0) a.dlast[(size_t)chunk * D + 16 * kt + r] = part;
}

// ------------------------------------------------------------------------------------
// bwd_state_rc: the reductions of bwd_state with the states recomputed from checkpoints.
// One workgroup of NWW waves per (batch, head, block of K = ckpt chunks, group of NWW key
// tiles); wave w owns key tile kt = grp NWW + w (key rows 16 kt .. 16 kt + 15) over all value
// columns, with that slice of the state in registers in the MFMA result layout (lane (r, g) of
// block kb holds h[16 kt + 4 g + e][16 kb + r], which is lane l of FA(h^T) block (kb, kt), the
// checkpoint's layout).  Per chunk c of the block and value block kb:
//   reductions   as bwd_state (dQg^T, dWp^T, dKg^T tiles (kt, ti) over kb; sum_v dh_next h)
//                with h_pre block (kt, kb) = the register block, turned into the B-operand
//                layout by a per-wave LDS transpose;
//   state step   (all chunks of the block but the last) h[kt, kb] = state_update(h, gamma,
//                sum_u Kg^T[kt, u] v_new[u, kb]): the forward scan's update with the same
//                operands in the same MFMA order, so the recomputed state is the forward's bit
//                for bit.  Given v_new (stored), each key tile's rows step on their own: no
//                exchange between waves.
// A operands of one kb are staged once per workgroup in LDS (double-buffered, one barrier per
// kb; the staging pipeline runs across chunk boundaries): s dO, -dv_new, v_new in the A-operand
// layout (transposed on the way in) and v_new as stored (FA(v_new^T) blocks, which are the
// B operands of Kg^T v_new).
// ------------------------------------------------------------------------------------
template <int D, int NWW, int B3, int DOT>
__global__ __launch_bounds__(NWW * WAVE) __attribute__((amdgpu_waves_per_eu(2))) void bwd_state_rc_kernel(
    BwdStateRcArgs a) {
  constexpr int NKB = D / 16, NKT = D / 16, NG = NKT / NWW;
  constexpr int SLAB = 16 * WAVE;                // float4 staged per value block
  constexpr int NST = 3;                         // float4 loaded per thread per value block
  static_assert(NWW == 4, "staging: wave w loads token tile w of each of the three operands");
  static_assert(NKT % NWW == 0 && NKB % 2 == 0, "key tile groups, value block parity");
  __shared__ float4 sA[2 * SLAB];                // [buf][mat * 4 + tile][lane]
  __shared__ __attribute__((aligned(16))) float sTr[NWW * 16 * TRP];
  // Cfg::group = G > 1: the damped state h_d of the next part (its dWp uses it), [wave][kb][lane],
  // stepped through the parts as the forward scan does (K is a multiple of G: a block holds
  // whole big chunks)
  __shared__ float4 sHd[NWW * NKB * WAVE];
  const Cfg& cf = a.cfg;
  const int nc = a.nc;
  const int G = cf.group;
  const CkptBlocks cb(nc, a.ckpt, G);
  const int nblk = cb.nblk;
  const float inv_eps = G > 1 ? 1.f / cf.wy_eps : 0.f;
  // Work order: each XCD (blockIdx % 8) takes whole (batch, head)s, all their full blocks first
  // and then their remainder blocks, so that the short blocks are the ones left waiting for a
  // free slot; the two key-tile groups of a block, which stage the same operands, are adjacent
  // on one XCD.  When n_bh is not a multiple of 8: the same order over the whole grid.
  int grp, blk, bh;
  {
    const int nF = cb.nfull * NG, nR = (nblk - cb.nfull) * NG;
    const bool xcd = a.n_bh % 8 == 0;
    const int per = xcd ? a.n_bh / 8 : a.n_bh;                 // (batch, head)s per XCD
    const int x = xcd ? blockIdx.x % 8 : 0, p = xcd ? blockIdx.x / 8 : blockIdx.x;
    int bhl, r;
    if (p < per * nF) {
      bhl = p / nF;
      r = p % nF;
      blk = r / NG;
    } else {
      const int q = p - per * nF;
      bhl = q / nR;
      r = q % nR;
      blk = cb.nfull + r / NG;
    }
    grp = r % NG;
    bh = x * per + bhl;
  }
  const int c0 = cb.start(blk), c1 = c0 + cb.len(blk);
  const int w = wave_id(), kt = grp * NWW + w, l = lane_id(), r = l & 15, g = l >> 4;
  const float sc = cf.scale, clip = cf.clip;
  float* tr = sTr + w * 16 * TRP;
  auto chunk_idx = [&](int c) { return (size_t)bh * nc + c; };

  // staging: wave w loads and stages token tile ti = w of the value block's three A operands
  // (s dO, -dv_new, v_new), one float4 per lane each
  // wave-uniform base pointers plus unsigned 32-bit lane offsets, so that the loads take the
  // scalar-base form and no 64-bit per-lane address is kept live across the loop
  const unsigned lo_do = (unsigned)((r * D) + 4 * g), lo4 = 4u * (unsigned)l;
  auto fetch = [&](int c, int kb, float4 (&dst)[NST]) {
    const size_t tb = chunk_idx(c) * T * D, tio = ((size_t)bh * cf.seq_ld + (size_t)c * T) * D;
    dst[0] = ld4(sbase(a.dout + tio + (16 * w * D + 16 * kb)) + lo_do);
    dst[1] = ld4(sbase(a.dv_new_f + tb + frag_blk(w, kb, D)) + lo4);
    dst[2] = ld4(sbase(a.v_new_f + tb + frag_blk(kb, w, T)) + lo4);
  };
  auto put = [&](int buf, const float4 (&src)[NST]) {
    float4* base = sA + buf * SLAB;
    base[w * WAVE + l] = scale4(src[0], sc);
    base[(4 + w) * WAVE + l] = scale4(src[1], -1.f);
    // lane (r, g) holds v_new[16 w + 4 g + e][16 kb + r]: A-operand lane (4 g + e) + 16 (r / 4),
    // component r % 4; and as stored for the state step
    float* df = reinterpret_cast<float*>(base + (8 + w) * WAVE);
    const int o = 4 * (4 * g + 16 * (r >> 2)) + (r & 3);
    df[o] = src[2].x;
    df[o + 4] = src[2].y;
    df[o + 8] = src[2].z;
    df[o + 12] = src[2].w;
    base[(12 + w) * WAVE + l] = src[2];
  };
  auto dh_at = [&](int c, int kb) { return ld4(sbase(a.dh_next_f + chunk_idx(c) * D * D + frag_blk(kt, kb, D)) + lo4); };
  // EZ(part + 1) of chunk c (scan_bwd; Cfg::group), added to dh_next in its dKg; zero where
  // unused (no damping, or the last part of a big chunk)
  auto ez_at = [&](int c, int kb) {
    if (G == 1 || c % G == G - 1) return make_float4(0.f, 0.f, 0.f, 0.f);
    return ld4(sbase(a.ez_f + chunk_idx(c) * D * D + frag_blk(kt, kb, D)) + lo4);
  };

  f4 h[NKB];
  {
    const size_t hcb = ((size_t)bh * nblk + blk) * D * D;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const float4 x = ld4(sbase(a.hck_f + hcb + frag_blk(kb, kt, D)) + lo4);
      h[kb] = f4{x.x, x.y, x.z, x.w};
    }
  }
  float4 st[2][NST], dhb[2], ezb[2];
  fetch(c0, 0, st[0]);
  dhb[0] = dh_at(c0, 0);
  ezb[0] = ez_at(c0, 0);
  fetch(c0, 1, st[1]);
  dhb[1] = dh_at(c0, 1);
  ezb[1] = ez_at(c0, 1);
  put(0, st[0]);
  __syncthreads();

  for (int c = c0; c < c1; ++c) {
    const size_t ch = chunk_idx(c), tb = ch * T * D;
    const bool step = c + 1 < c1;
    const int pj = G > 1 ? c % G : 0;                // part of a damped big chunk
    const bool second = pj > 0;                      // dWp (the erase term) from h_d
    const bool dterm = pj > 0 && pj < G - 1;         // gamma's gradient through Delta
    float4 kga[4] = {}, gm = make_float4(0.f, 0.f, 0.f, 0.f);
    if (step) {
      // Kg^T block (kt, u) in the A-operand layout = FA(Kg) block (u, kt) transposed
#pragma unroll
      for (int u = 0; u < 4; ++u) kga[u] = wave_transpose16(tr, ld4(sbase(a.kg_f + tb + frag_blk(u, kt, D)) + lo4), r, g);
      gm = ld4(sbase(a.gl + ch * D + 16 * kt) + 4 * g);
    }
    f4 acc[3][4];
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) acc[m][ti] = f4{0.f, 0.f, 0.f, 0.f};
    float part = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int pb = kb & 1;
      const float4 hp = wave_transpose16(tr, f4_to_float4(h[kb]), r, g);
      const float4 hpw = second ? wave_transpose16(tr, sHd[(w * NKB + kb) * WAVE + l], r, g) : hp;
      // this value block's dh_next and EZ, taken before the prefetch below refills their slots
      const float4 dhc = dhb[pb], ezc = ezb[pb];
      const float4 dhk = add4(dhc, ezc);
      {
        // two value blocks ahead, across the chunk boundary
        const int kn = kb + 2 < NKB ? kb + 2 : kb + 2 - NKB, cn = kb + 2 < NKB ? c : c + 1;
        if (cn < c1) {
          fetch(cn, kn, st[pb]);
          dhb[pb] = dh_at(cn, kn);
          ezb[pb] = ez_at(cn, kn);
        }
      }
      const float4* cur = sA + pb * SLAB;
      // operands of token tile ti + 1 are read while tile ti's MFMAs issue; the fences keep
      // the compiler from hoisting every read of the block (64 VGPRs) above the first MFMA
      float4 o0 = cur[l], o1 = cur[4 * WAVE + l], o2 = cur[8 * WAVE + l];
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        float4 n0 = o0, n1 = o1, n2 = o2;
        if (ti < 3) {
          n0 = cur[(ti + 1) * WAVE + l];
          n1 = cur[(5 + ti) * WAVE + l];
          n2 = cur[(9 + ti) * WAVE + l];
        }
        mma16<B3>(acc[0][ti], o0, hp);
        mma16<B3>(acc[1][ti], o1, hpw);
        mma16<B3>(acc[2][ti], o2, dhk);
        __builtin_amdgcn_sched_barrier(0);
        o0 = n0;
        o1 = n1;
        o2 = n2;
      }
      part = fmaf(dhc.x, hp.x, part);
      part = fmaf(dhc.y, hp.y, part);
      part = fmaf(dhc.z, hp.z, part);
      part = fmaf(dhc.w, hp.w, part);
      if (dterm) {
        // sum_v EZ(pj + 1) Delta(pj), Delta = (h - h_d) / eps (gdn2_kernels.hpp, Cfg::group)
        part = fmaf(ezc.x, (hp.x - hpw.x) * inv_eps, part);
        part = fmaf(ezc.y, (hp.y - hpw.y) * inv_eps, part);
        part = fmaf(ezc.z, (hp.z - hpw.z) * inv_eps, part);
        part = fmaf(ezc.w, (hp.w - hpw.w) * inv_eps, part);
      }
      if (step) {
        // the forward scan's Kg^T v_new chain (gdn2_scan.hip), the same MFMAs in the same order
        f4 hn = {0.f, 0.f, 0.f, 0.f};
        mma_chain<DOT, 4>(hn, 0, [&](int u) { return kga[u]; }, [&](int u) { return cur[(12 + u) * WAVE + l]; });
        drain(hn);
        const float gmv[4] = {gm.x, gm.y, gm.z, gm.w};
        if (G > 1 && pj < G - 1) {
          // the forward scan's damped state of the next part (gdn2_scan.hip), bit for bit:
          // h_d(pj + 1) = san(e^gamma h_d(pj) + (1 - eps) Kg^T v_new), h_d(0) = h
          const float ome = cf.ome;
          float4& hd = sHd[(w * NKB + kb) * WAVE + l];
          const float4 b0 = pj == 0 ? f4_to_float4(h[kb]) : hd;
          hd = make_float4(state_update(b0.x, gmv[0], ome * hn[0], clip), state_update(b0.y, gmv[1], ome * hn[1], clip),
                           state_update(b0.z, gmv[2], ome * hn[2], clip), state_update(b0.w, gmv[3], ome * hn[3], clip));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) h[kb][e] = state_update(h[kb][e], gmv[e], hn[e], clip);
      }
      if (kb + 1 < NKB || c + 1 < c1) put(pb ^ 1, st[pb ^ 1]);     // the next value block
      __syncthreads();
    }
    drain(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
    drain(acc[1][0], acc[1][1], acc[1][2], acc[1][3]);
    drain(acc[2][0], acc[2][1], acc[2][2], acc[2][3]);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const size_t o = tb + frag_blk(kt, ti, T);
      stg4(sbase(a.dqg + o) + lo4, f4_to_float4(acc[0][ti]));
      stg4(sbase(a.dwp + o) + lo4, f4_to_float4(acc[1][ti]));
      stg4(sbase(a.dkg + o) + lo4, f4_to_float4(acc[2][ti]));
    }
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
    if (g == 0) sbase(a.dlast + ch * D + 16 * kt)[r] = part;
  }
}

// ------------------------------------------------------------------------------------
// bwd_wy: one workgroup (8 waves) per chunk.
//
// Output ownership: wave w owns column strip s = w % (D/16) (columns 16 s .. 16 s + 15) and
// NTW row tiles of it.  Lane l = n + 16 g works on column 16 s + n and rows 16 t + 4 g + e
// (e = 0..3) of every row tile t: the MFMA accumulator layout, which is also the B-operand
// layout, so the per-element factors of B4 (legs, q/k/b) computed once per lane feed both
// the MFMA operands and the element-wise updates.
//
// Phases (LDS: gc | X1 | X2 | A | dAqk | dA/dAkk | column partial sums):
//   P1 dAqk = (dO v_new^T) * causal                 X1 = v_new, X2 = dO              (mega.py:32)
//   P2 dA = san(dWp kb^T + dv_new (w v)^T)           X1 = kb / w v, X2 = dWp / dv_new (mega.py:41)
//      and per owned tile dwv = A^T dv_new                                          (mega.py:42)
//   P3 tmp = san(dA A^T)                               X2 = tmp, X1 = dwv           (mega.py:43)
//   dw = san(dwv v), dv = san(dwv w) as row-major items, stored here           (mega.py:57-58)
//   P4 dAkk = san(-(1-eps) A^T tmp) * strict                                       (mega.py:44)
//   B4 VJP of the two-level scores, piece by piece (owned tiles, registers)   (b4.py:45-97)
//   per owned tile: dkb = A^T dWp (mega.py:42), the gate gradients
//   dq3 / dk3 / db3 / dgc3 and the combine with B4                           (mega.py:45-59)
//   B5 dg = reverse cumsum of dgc3 + dgc4                                            (mega.py:53)
// ------------------------------------------------------------------------------------
template <int D>
struct BwdWyLayout {
  // X1 and X2 (T x LD each) are arrays of their own (X2 rounded up to whole DMA windows for the
  // persistent kernel, which fills both by LDS DMA).
  static constexpr int LD = D + 4, LT = T + 4;
  static constexpr int OFF_G = 0, OFF_A = T * LD, OFF_DAQ = OFF_A + T * LT, OFF_DA = OFF_DAQ + T * LT;
  static constexpr int OFF_COL = OFF_DA + T * LT;
  static constexpr int TOTAL = OFF_COL + 8 * 16;
};

// Tiles of a T x D output owned by wave w: column strip w % (D/16); row tiles
// w / (D/16) + m * (8 / (D/16)), m = 0..NTW-1.
template <int D>
struct Strip {
  static constexpr int NS = D / 16, NTW = (T / 16) * NS / 8, STEP = 8 / NS;
  __device__ static int strip(int w) { return w % NS; }
  __device__ static int rtile(int w, int m) { return w / NS + m * STEP; }
};

// x[t] for a runtime t in [0, 4) as selects over constant indices (no dynamic register
// indexing, which would move the array to scratch memory)
__device__ __forceinline__ float sel4(float a0, float a1, float a2, float a3, int t) {
  return t == 0 ? a0 : (t == 1 ? a1 : (t == 2 ? a2 : a3));
}
__device__ __forceinline__ float4 pick4(const float4 (&x)[4], int t) {
  return make_float4(sel4(x[0].x, x[1].x, x[2].x, x[3].x, t), sel4(x[0].y, x[1].y, x[2].y, x[3].y, t),
                     sel4(x[0].z, x[1].z, x[2].z, x[3].z, t), sel4(x[0].w, x[1].w, x[2].w, x[3].w, t));
}

// STD: the pieces are the standard geometry's (bt = score_bs = 64, bs2 = 32), see std_pieces().
// EM: elementwise pieces, a compile-time choice, so that the other kernels carry no trace of
// the elementwise loops (whose live ranges otherwise push registers into scratch):
//   EM_NONE  every piece on MFMA;
//   EM_LEAN  the lean diagonal (cfg.diag): its diagonal-block pieces elementwise and exact;
//   EM_MIX   pieces narrower than a 16 x 16 tile (bs2 = 8): every piece elementwise, with its
//            legs (or, with the lean diagonal, the diagonal blocks exactly).
enum { EM_NONE = 0, EM_LEAN = 1, EM_MIX = 2 };
template <int D, int B3, bool STD, int EM>
__global__ __launch_bounds__(512) void bwd_wy_kernel(BwdWyArgs a) {
  constexpr bool ELEM = EM != EM_NONE;
  static_assert(!(STD && ELEM), "the standard piece list is the BTL one");
  using Lay = BwdWyLayout<D>;
  using St = Strip<D>;
  constexpr int LD = Lay::LD, LT = Lay::LT, NT = 512, NW = 8, NTW = St::NTW, NKB = D / 16;
  // RT_STATIC: every wave owns a whole column strip (D = 128), rt == m for every wave.
  // PERSIST: one workgroup per CU walks the chunks blockIdx.x, + gridDim.x, ...; the next
  // chunk's prologue operands are fetched during this chunk's B4 and gate phase (below).
  // Other instantiations run the body once (one workgroup per chunk).
  constexpr bool RT_STATIC = St::NS == NW, PERSIST = RT_STATIC && !ELEM;
  // X2 as DMA windows of 256 floats, a whole number per wave (the tail past T x LD is slack)
  constexpr int X2_WIN = PERSIST ? (T * LD / 256 + NW - 1) / NW * NW : (T * LD + 255) / 256;
  __shared__ __attribute__((aligned(16))) float smem[Lay::TOTAL];
  __shared__ __attribute__((aligned(16))) float sX1[T * LD];
  __shared__ __attribute__((aligned(16))) float sX2[X2_WIN * 256];
  float* sG = smem + Lay::OFF_G;
  float* sA = smem + Lay::OFF_A;
  float* sDAq = smem + Lay::OFF_DAQ;
  float* sDA = smem + Lay::OFF_DA;
  float* sColP = smem + Lay::OFF_COL;
  constexpr int NIT = T * D / 4 / NT, NIA = T * T / 4 / NT;
  float4 xa[NIA], xg[4];                            // PERSIST: next chunk's A and g column
  const BwdWyArgs& a0 = a;

  for (int chunk = blockIdx.x, first = 1; first || (PERSIST && chunk < a0.n_chunks); chunk += gridDim.x, first = 0) {
  // In the loop the arguments are read through an opaque pointer to the kernel argument block
  // and the lane indices come from an opaque copy of threadIdx.x, both fresh in every
  // iteration: the argument pointers and the many lane-dependent addresses are then recomputed
  // where they are used, instead of being hoisted out of the loop and held in registers.
  const auto& a = *kernarg_fresh<BwdWyArgs>(PERSIST);
  const auto& cf = a.cfg;
  const float clip = cf.clip, scale = cf.scale;
  int tid_;
  asm volatile("" : "=v"(tid_) : "0"((int)threadIdx.x));
  const int tid = tid_ & (NT - 1);                  // the range the optimiser knew for threadIdx.x
  const int wv = __builtin_amdgcn_readfirstlane(tid / WAVE), l = tid & (WAVE - 1), r = l & 15, g = l >> 4;
  const int strip = St::strip(wv), dcol = 16 * strip + r;
  auto owned = [&](int t) { return t >= St::rtile(wv, 0) && (t - St::rtile(wv, 0)) % St::STEP == 0; };

  // x[16 t + 4 g + e][dcol], e = 0..3: this lane's column at the rows of row tile t
  auto col4 = [&](const float* __restrict__ x, int t) {
    const float* p = x + (16 * t + 4 * g) * D + dcol;
    return make_float4(p[0], p[D], p[2 * D], p[3 * D]);
  };
  // the same for a T x D tensor stored as FA(x^T): one float4 of block (strip, t)
  auto fcol4 = [&](const float* __restrict__ x, int t) { return ldg4(x + frag_blk(strip, t, T) + 4 * l); };

  // Item f of a row-major input is float4 f; item f of a FRAG(x^T) (v_new, dWp) or FRAG(x)
  // (dv_new) input is float4 f as well, placed into the row-major tile by put_fragT / put_frag.
  auto put_frag = [&](float* dst, const float4& x, int f) {
    const int lane = f & 63, blk = f >> 6;
    st4(dst + (16 * (blk / NKB) + (lane & 15)) * LD + 16 * (blk % NKB) + 4 * (lane >> 4), x);
  };
  auto put_fragT = [&](float* dst, const float4& x, int f) {
    const int lane = f & 63, blk = f >> 6;
    const int n = 16 * (blk >> 2) + (lane & 15), m = 16 * (blk & 3) + 4 * (lane >> 4);
    dst[(m + 0) * LD + n] = x.x;
    dst[(m + 1) * LD + n] = x.y;
    dst[(m + 2) * LD + n] = x.z;
    dst[(m + 3) * LD + n] = x.w;
  };

  // PERSIST prologue operands of a chunk, fetched while the previous chunk is in B4:
  //   v_new -> X1 by LDS DMA (global_load_lds_dwordx4, no registers): its 32 fragment blocks
  //     FA(v_new^T) as they are stored, except that within a block quad q (lane q of the
  //     fragment) lands in slot sig(q) = (q & 48) | ((q + (q >> 4)) & 15), which makes P1's
  //     gathers of v_new rows free of bank conflicts (vnb below);
  //   dO -> X2 by LDS DMA in the padded row-major layout: X2 is X2_WIN windows of 256 floats,
  //     five per wave, lane i of window u fetches the quad at float 256 u + 4 i, and a quad in
  //     a row's padding or past the last row fetches row 0 (never read); every wave issues the
  //     same number of DMAs, so the compiler can count them in its waits;
  //   A and this lane's g column (the in-wave cumsum below) in registers.
  static_assert((D / 16) * (T / 16) % NW == 0 && X2_WIN * 256 >= T * LD, "DMA windows");
  auto fetch_dma = [&](int ch) {
    const float* vsrc = a.v_new_f + (size_t)ch * T * D;
    const size_t cio = io_off<D>(cf, ch);
    const int qi = (l & 48) | (((l & 15) - (l >> 4)) & 15);        // sig^-1(lane)
#pragma unroll
    for (int j = 0; j < (D / 16) * (T / 16) / NW; ++j) {
      const int blk = wv + NW * j;
      lds_dma16(vsrc + blk * 256 + 4 * qi, sX1 + blk * 256);
    }
#pragma unroll
    for (int j = 0; j < X2_WIN / NW; ++j) {
      const int u = wv + NW * j, f = 256 * u + 4 * l, row = f / LD, col = f - row * LD;
      lds_dma16(a.dout + cio + (row < T && col < D ? row * D + col : 0), sX2 + 256 * u);
    }
  };
  auto fetch_regs = [&](int ch) {
    const size_t cio = io_off<D>(cf, ch);
#pragma unroll
    for (int it = 0; it < NIA; ++it) xa[it] = ldg4(a.A + (size_t)ch * T * T + 4 * (tid + it * NT));
    const float* gp = a.g + cio + 4 * g * D + dcol;
#pragma unroll
    for (int t = 0; t < 4; ++t) xg[t] = make_float4(gp[16 * t * D], gp[(16 * t + 1) * D], gp[(16 * t + 2) * D], gp[(16 * t + 3) * D]);
  };
  if constexpr (PERSIST) {
    if (first) fetch_dma(chunk);
    fetch_regs(chunk);
  }
  const size_t tb = (size_t)chunk * T * D, sb = (size_t)chunk * T * T, tio = io_off<D>(cf, chunk);
  const float* __restrict__ q = a.q + tio;
  const float* __restrict__ k = a.k + tio;
  const float* __restrict__ b = a.b + tio;
  const float* __restrict__ w = a.w + tio;
  const float* __restrict__ v = a.v + tio;
  const float* __restrict__ dout = a.dout + tio;
  const float* __restrict__ dwp = a.dwp + tb;
  const int next = chunk + gridDim.x;

  // X1 = v_new, X2 = dO, sA = A, sG = gc.  Non-persistent: every load is issued before the
  // cumsum waits for its g, one memory round trip for the whole prologue.  Persistent: X1 and X2
  // arrived by DMA during the previous chunk's B4 (the first chunk's are waited for here), and
  // A and g, loaded above, are only stored after P1, which reads neither: their round trip runs
  // under P1's MFMAs.
  if constexpr (PERSIST) {
    if (first) __builtin_amdgcn_s_waitcnt(WAIT_VMCNT0);
  } else {
    float4 xvn[NIT], xdo[NIT], xa[NIA];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      xvn[it] = ldg4(a.v_new_f + tb + 4 * (tid + it * NT));
      xdo[it] = ldg4(dout + 4 * (tid + it * NT));
    }
#pragma unroll
    for (int it = 0; it < NIA; ++it) xa[it] = ldg4(a.A + sb + 4 * (tid + it * NT));
    chunk_cumsum<D, LD, NT, true>(a.g + tio, sG);
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int f = tid + it * NT;
      put_fragT(sX1, xvn[it], f);
      st4(sX2 + (f / (D / 4)) * LD + 4 * (f % (D / 4)), xdo[it]);
    }
#pragma unroll
    for (int it = 0; it < NIA; ++it) {
      const int f = tid + it * NT;
      st4(sA + (f >> 4) * LT + 4 * (f & 15), xa[it]);
    }
  }
  __syncthreads();

  // The P2 operands' global loads are spread between P1's MFMAs (a burst of loads stalls the
  // issuing wave while the CU's memory path is busy).  b, k and dWp arrive as this lane's
  // column at the rows of the four row tiles (the layout B4, the dkb chain and the gates use,
  // so they stay in registers to the end); w, v, dv_new as row-major / fragment items, which
  // also serve dw / dv after P2.  Every input is read once.
  float4 kv[4], bv[4], dwpc[4];
  float4 xw[NIT], xv[NIT], xdv[NIT];
  constexpr int NRT = T / 16;
  auto prefetch = [&](int item) {
    if (item < 3 * NRT) {
      if (item < NRT) bv[item] = col4(b, item);
      else if (item < 2 * NRT) kv[item - NRT] = col4(k, item - NRT);
      else dwpc[item - 2 * NRT] = fcol4(dwp, item - 2 * NRT);
      return;
    }
    const int arr = (item - 3 * NRT) / NIT, it = (item - 3 * NRT) % NIT, f = tid + it * NT;
    if (arr == 0) xw[it] = ldg4(w + 4 * f);
    else if (arr == 1) xv[it] = ldg4(v + 4 * f);
    else xdv[it] = ldg4(a.dv_new_f + tb + 4 * f);
  };

  // P1: dAqk = (dO v_new^T) * causal; 16 tiles, two per wave.  Its MFMAs carry the loads of
  // b, k and dWp (staged right after it); w, v and dv_new go out during P2a, which stages them
  // next: each phase's loads then overlap the MFMAs of the phase before their use.
  static_assert(NW == 8, "P1 assumes two dAqk tiles per wave");
  constexpr int NITEMS1 = 3 * NRT, NITEMS2 = 3 * NIT, NSLOT = 2 * NKB;
#pragma unroll
  for (int m2 = 0; m2 < 2; ++m2) {
    const int t = wv + NW * m2, ti = t >> 2, tj = t & 3;
    const float* ar = sX2 + (16 * ti + r) * LD + 4 * g;
    const float* br = sX1 + (16 * tj + r) * LD + 4 * g;
    // B operand v_new[16 tj + r][16 kb + 4 g + e]: row-major X1, or (PERSIST) the swizzled
    // fragment blocks: lane q = 4 g + e + 16 (r >> 2), element r & 3 of block (kb, tj)
    const float* bq = sX1 + 64 * (r >> 2) + (r & 3);
    auto vnb = [&](int kb) {
      if constexpr (!PERSIST) return ld4(br + 16 * kb);
      const float* p = bq + (4 * kb + tj) * 256;
      return make_float4(p[4 * ((4 * g + (r >> 2)) & 15)], p[4 * ((4 * g + 1 + (r >> 2)) & 15)],
                         p[4 * ((4 * g + 2 + (r >> 2)) & 15)], p[4 * ((4 * g + 3 + (r >> 2)) & 15)]);
    };
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    constexpr int KSTEP = B3 == DOT_HIGHEST ? 1 : 2;      // bf16: two k blocks per MFMA
#pragma unroll
    for (int kb = 0; kb < NKB; kb += KSTEP) {
      if constexpr (KSTEP == 1) mma16<B3>(acc, ld4(ar + 16 * kb), vnb(kb));
      else mma32<B3>(acc, ld4(ar + 16 * kb), vnb(kb), ld4(ar + 16 * kb + 16), vnb(kb + 1));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int sl = m2 * NKB + kb; sl < m2 * NKB + kb + KSTEP; ++sl)
#pragma unroll
        for (int item = NITEMS1 * sl / NSLOT; item < NITEMS1 * (sl + 1) / NSLOT; ++item) prefetch(item);
      __builtin_amdgcn_sched_barrier(0);
    }
    drain(acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * ti + 4 * g + e, j = 16 * tj + r;
      sDAq[i * LT + j] = j <= i ? acc[e] : 0.f;
    }
  }
  if constexpr (PERSIST) {
    // A from registers; gc of this wave's columns by an in-wave cumsum that adds in the order
    // chunk_cumsum does (runs of four rows, then the totals of the runs above in order), so gc
    // is bit-identical to every other kernel's.  Run s = 4 t + g is this lane's row tile t.
#pragma unroll
    for (int it = 0; it < NIA; ++it) {
      const int f = tid + it * NT;
      st4(sA + (f >> 4) * LT + 4 * (f & 15), xa[it]);
    }
    float xr[4][4], offt[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      xr[t][0] = xg[t].x;
      xr[t][1] = xr[t][0] + xg[t].y;
      xr[t][2] = xr[t][1] + xg[t].z;
      xr[t][3] = xr[t][2] + xg[t].w;
    }
    float run = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2) {
      const int t2 = s2 >> 2, g2 = s2 & 3;
      offt[t2] = g == g2 ? run : offt[t2];
      run = run + __shfl(xr[t2][3], r + 16 * g2);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) sG[(16 * t + 4 * g + e) * LD + dcol] = offt[t] + xr[t][e];
  }
  __syncthreads();

  // P2: dA = san(dWp kb^T + dv_new (w v)^T), the two products with operands staged in turn:
  //     X1 = kb = b k e^{min(gc,0)}, X2 = dWp; then X1 = w v, X2 = dv_new (for dwv)
  // X1 = kb and X2 = dWp at this wave's column strip and owned row tiles (every element
  // written once)
#pragma unroll
  for (int t = 0; t < NRT; ++t) {
    if (!owned(t)) continue;
    const float bb[4] = {bv[t].x, bv[t].y, bv[t].z, bv[t].w}, kk[4] = {kv[t].x, kv[t].y, kv[t].z, kv[t].w};
    const float dd[4] = {dwpc[t].x, dwpc[t].y, dwpc[t].z, dwpc[t].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * t + 4 * g + e;
      sX1[i * LD + dcol] = (bb[e] * kk[e]) * exp_nonpos(sG[i * LD + dcol]);
      sX2[i * LD + dcol] = dd[e];
    }
  }
  __syncthreads();
  f4 accA[2];
#pragma unroll
  for (int m2 = 0; m2 < 2; ++m2) {
    const int t = wv + NW * m2, ti = t >> 2, tj = t & 3;
    const float* ar = sX2 + (16 * ti + r) * LD + 4 * g;
    const float* br = sX1 + (16 * tj + r) * LD + 4 * g;
    accA[m2] = f4{0.f, 0.f, 0.f, 0.f};
    constexpr int KSTEP = B3 == DOT_HIGHEST ? 1 : 2;      // the block steps of mma_chain<B3, NKB>
#pragma unroll
    for (int kb = 0; kb < NKB; kb += KSTEP) {
      if constexpr (KSTEP == 1) mma16<B3>(accA[m2], ld4(ar + 16 * kb), ld4(br + 16 * kb));
      else mma32<B3>(accA[m2], ld4(ar + 16 * kb), ld4(br + 16 * kb), ld4(ar + 16 * kb + 16), ld4(br + 16 * kb + 16));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int sl = m2 * NKB + kb; sl < m2 * NKB + kb + KSTEP; ++sl)
#pragma unroll
        for (int item = NITEMS2 * sl / NSLOT; item < NITEMS2 * (sl + 1) / NSLOT; ++item) prefetch(NITEMS1 + item);
      __builtin_amdgcn_sched_barrier(0);
    }
    drain(accA[m2]);
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int f = tid + it * NT, i = f / (D / 4), d = 4 * (f % (D / 4));
    st4(sX1 + i * LD + d, mul4(xw[it], xv[it]));
    put_frag(sX2, xdv[it], f);
  }
  __syncthreads();
#pragma unroll
  for (int m2 = 0; m2 < 2; ++m2) {
    const int t = wv + NW * m2, ti = t >> 2, tj = t & 3;
    const float* ar = sX2 + (16 * ti + r) * LD + 4 * g;
    const float* br = sX1 + (16 * tj + r) * LD + 4 * g;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    mma_chain<B3, NKB>(acc, 0, [&](int kb) { return ld4(ar + 16 * kb); }, [&](int kb) { return ld4(br + 16 * kb); });
    drain(acc);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      sDA[(16 * ti + 4 * g + e) * LT + 16 * tj + r] = sanitize(accA[m2][e] + acc[e], clip);
  }
  // dwv = A^T dv_new on the owned tiles (mega.py:42; A^T is upper triangular, so row tile rt
  // only sees k blocks >= rt).  It needs no B4 result, so dw and dv leave before B4 (their
  // stores overlap P3 / P4 / B4) and the gate phase keeps only the dkb chain.
  f4 dwv[NTW];
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    const int rt = St::rtile(wv, m);
    auto acol = [&](int kb) {
      const float* ac = sA + (16 * kb + 4 * g) * LT + 16 * rt + r;
      return make_float4(ac[0], ac[LT], ac[2 * LT], ac[3 * LT]);
    };
    auto pcol = [&](int kb) {
      const float* pv = sX2 + (16 * kb + 4 * g) * LD + dcol;
      return make_float4(pv[0], pv[LD], pv[2 * LD], pv[3 * LD]);
    };
    dwv[m] = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (B3 == DOT_HIGHEST) {
#pragma unroll
      for (int kb = RT_STATIC ? m : 0; kb < 4; ++kb) mma16<B3>(dwv[m], acol(kb), pcol(kb));
    } else {
      mma_chain<B3, 4>(dwv[m], RT_STATIC ? m : 0, acol, pcol);
    }
    drain(dwv[m]);
  }
  __syncthreads();

  // q of this lane's column at the rows of all four row tiles (B4 and the gates), loaded
  // here so that it arrives during P3 / P4
  float4 qv[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) qv[t] = col4(q, t);

  // dwv -> X1 (row-major), read back below as the row-major items of w and v
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    const int rt = St::rtile(wv, m);
#pragma unroll
    for (int e = 0; e < 4; ++e) sX1[(16 * rt + 4 * g + e) * LD + dcol] = dwv[m][e];
  }

  // P3: tmp = san(dA A^T) into X2 (as T x LT; dv_new is done with).  A is lower triangular, so
  // column tile tj only sees k blocks <= tj; tj is wave-uniform, and a switch keeps each chain
  // straight-line with a compile-time length.
  float* sTmp = sX2;
  for (int t = wv; t < 16; t += NW) {
    const int ti = t >> 2, tj = t & 3;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    auto fa = [&](int kb) { return ld4(sDA + (16 * ti + r) * LT + 16 * kb + 4 * g); };
    auto fb = [&](int kb) { return ld4(sA + (16 * tj + r) * LT + 16 * kb + 4 * g); };
    // each case drains its own chain: the accumulator is read (merged at the join) only after
    switch (tj) {
      case 0: mma_chain<B3, 1>(acc, 0, fa, fb); drain(acc); break;
      case 1: mma_chain<B3, 2>(acc, 0, fa, fb); drain(acc); break;
      case 2: mma_chain<B3, 3>(acc, 0, fa, fb); drain(acc); break;
      default: mma_chain<B3, 4>(acc, 0, fa, fb); drain(acc); break;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) sTmp[(16 * ti + 4 * g + e) * LT + 16 * tj + r] = sanitize(acc[e], clip);
  }
  __syncthreads();

  // dw = san(dwv v), dv = san(dwv w) (mega.py:57-58), row-major items, one float4 store each.
  // q (for B4) is waited for here, before the first store (see the gate phase's loads below).
  __builtin_amdgcn_s_waitcnt(WAIT_VMCNT0);
  float* __restrict__ o_dw = a.dw + tio;
  float* __restrict__ o_dv = a.dv + tio;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int f = tid + it * NT, i = f / (D / 4), d = 4 * (f % (D / 4));
    const float4 x = ld4(sX1 + i * LD + d);
    stg4(o_dw + i * D + d, san4(mul4(x, xv[it]), clip));
    stg4(o_dv + i * D + d, san4(mul4(x, xw[it]), clip));
  }

  // P4: dAkk = san(-(1-eps) A^T tmp) * strict into sDA; tiles above the diagonal are zero
  for (int t = wv; t < 16; t += NW) {
    const int ti = t >> 2, tj = t & 3;
    float ov[4] = {0.f, 0.f, 0.f, 0.f};
    if (tj <= ti) {
      // the blocks kb < ti of A^T are exact zeros: the chain starts at ti (wave-uniform; a
      // switch keeps it straight-line with a compile-time start)
      f4 acc = {0.f, 0.f, 0.f, 0.f};
      auto fa = [&](int kb) {
        const float* ac = sA + (16 * kb + 4 * g) * LT + 16 * ti + r;
        return make_float4(ac[0], ac[LT], ac[2 * LT], ac[3 * LT]);
      };
      auto fb = [&](int kb) {
        const float* tc = sTmp + (16 * kb + 4 * g) * LT + 16 * tj + r;
        return make_float4(tc[0], tc[LT], tc[2 * LT], tc[3 * LT]);
      };
      switch (ti) {
        case 0: mma_chain<B3, 4>(acc, 0, fa, fb); drain(acc); break;
        case 1: mma_chain<B3, 4>(acc, 1, fa, fb); drain(acc); break;
        case 2: mma_chain<B3, 4>(acc, 2, fa, fb); drain(acc); break;
        default: mma_chain<B3, 4>(acc, 3, fa, fb); drain(acc); break;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ov[e] = (16 * tj + r < 16 * ti + 4 * g + e) ? sanitize(-acc[e] * cf.ome, clip) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) sDA[(16 * ti + 4 * g + e) * LT + 16 * tj + r] = ov[e];
  }
  __syncthreads();

  // PERSIST: X1 and X2 are free from here on; the next chunk's v_new and dO start now, to
  // land during B4, and are waited for after it.
  if constexpr (PERSIST)
    if (next < a.n_chunks) fetch_dma(next);

  // Global operands of the gate phase, all issued before the phase's first store (the memory
  // counter is in order and covers stores too, so a load issued after a store would wait for
  // it): here, to arrive during B4, with fp32 products; after B4 with bf16 ones, whose B4
  // holds more registers.
  const float* __restrict__ dqgp = a.dqg + tb;
  const float* __restrict__ dkgp = a.dkg + tb;
  float4 dqg4s[NTW], dkg4s[NTW];
  auto gate_loads = [&]() {
#pragma unroll
    for (int m = 0; m < NTW; ++m) {
      dqg4s[m] = fcol4(dqgp, St::rtile(wv, m));
      dkg4s[m] = fcol4(dkgp, St::rtile(wv, m));
    }
  };
  if constexpr (B3 == DOT_HIGHEST) gate_loads();

  // B4: VJP of the two-level scores on the owned tiles (b4.py:45-97)
  f4 dq4[NTW], dbk4[NTW], dk4[NTW], dgc4[NTW];
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    dq4[m] = f4{0.f, 0.f, 0.f, 0.f};
    dbk4[m] = dq4[m];
    dk4[m] = dq4[m];
    dgc4[m] = dq4[m];
  }
  const bool lean = ELEM && cf.diag == DIAG_LEAN;
  auto elementwise = [&](const Piece& pc) { return ELEM && ((lean && pc.kind != 0) || pc.P < 16); };
  // this lane's block anchors of the kind-2 pieces (bs2 > 64), in this part's gc frame
  float ar = 0.f, az = 0.f;
  if (a.anc) {
    ar = a.anc[(size_t)chunk * 2 * D + dcol];
    az = a.anc[(size_t)chunk * 2 * D + D + dcol];
  }
  // One piece of the two-level score factorisation; with the standard geometry the three
  // pieces are compile-time constants, so every branch and index below folds away.
  auto b4_piece = [&](const Piece pc) __attribute__((always_inline)) {
    const int nb = pc.P / 16, tr0 = pc.row0 / 16, tc0 = pc.col0 / 16;
    // legs at this lane's positions; qt = q ra, bkt = (b k) ra over the piece rows,
    // kt = k cb over the piece columns (k blocks of 16)
    float4 ra[2], cbl[2], qt[2], bkt[2], kt[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int ti = tr0 + (kb < nb ? kb : 0), tj = tc0 + (kb < nb ? kb : 0);
      float rv[4], cv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        rv[e] = piece_row_leg(pc, sG, LD, 16 * ti + 4 * g + e, dcol, ar, az);
        cv[e] = piece_col_leg(pc, sG, LD, 16 * tj + 4 * g + e, dcol, ar, az);
      }
      ra[kb] = make_float4(rv[0], rv[1], rv[2], rv[3]);
      cbl[kb] = make_float4(cv[0], cv[1], cv[2], cv[3]);
      qt[kb] = mul4(pick4(qv, ti), ra[kb]);
      bkt[kb] = mul4(mul4(pick4(bv, ti), pick4(kv, ti)), ra[kb]);
      kt[kb] = mul4(pick4(kv, tj), cbl[kb]);
    }
    // A piece on the diagonal (row0 == col0) of 2 x 2 tiles has its upper tile (rows of tile 0,
    // columns of tile 1) exactly zero in dAqk (causal) and dAkk (strict): the row chain of row
    // tile 0 and the column chain of column tile 1 skip it.
    const bool diag_sq = pc.row0 == pc.col0;
    // rows of the piece: dq, dbk, dgc
    for (int rb = 0; rb < nb; ++rb) {
      const int ti = tr0 + rb;
      if (!owned(ti)) continue;
      f4 dqt = {0.f, 0.f, 0.f, 0.f}, dbt = {0.f, 0.f, 0.f, 0.f};
      const float* pq = sDAq + (16 * ti + r) * LT + pc.col0 + 4 * g;
      const float* pk = sDA + (16 * ti + r) * LT + pc.col0 + 4 * g;
      if (nb == 2 && !(diag_sq && rb == 0)) {          // whole chains per branch, each ending in drain()
        mma16<DOT_HIGHEST>(dqt, ld4(pq), kt[0]);
        mma16<DOT_HIGHEST>(dbt, ld4(pk), kt[0]);
        mma16<DOT_HIGHEST>(dqt, ld4(pq + 16), kt[1]);
        mma16<DOT_HIGHEST>(dbt, ld4(pk + 16), kt[1]);
        drain(dqt, dbt);
      } else {
        mma16<DOT_HIGHEST>(dqt, ld4(pq), kt[0]);
        mma16<DOT_HIGHEST>(dbt, ld4(pk), kt[0]);
        drain(dqt, dbt);
      }
      const float4 rr = rb ? ra[1] : ra[0], qq = rb ? qt[1] : qt[0], bb = rb ? bkt[1] : bkt[0];
      const float rv[4] = {rr.x, rr.y, rr.z, rr.w}, qtv[4] = {qq.x, qq.y, qq.z, qq.w};
      const float btv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        if (St::rtile(wv, m) != ti) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = scale * dqt[e];
          dq4[m][e] += x * rv[e];
          dbk4[m][e] += dbt[e] * rv[e];
          dgc4[m][e] += x * qtv[e] + dbt[e] * btv[e];
        }
      }
    }
    // columns of the piece: dk, dgc
    for (int cb = 0; cb < nb; ++cb) {
      const int tj = tc0 + cb;
      if (!owned(tj)) continue;
      f4 k1 = {0.f, 0.f, 0.f, 0.f}, k2 = {0.f, 0.f, 0.f, 0.f};
      auto colop = [&](const float* base, int kb) {
        const float* p = base + (pc.row0 + 16 * kb + 4 * g) * LT + 16 * tj + r;
        return make_float4(p[0], p[LT], p[2 * LT], p[3 * LT]);
      };
      if (nb == 2 && diag_sq && cb == 1) {
        mma16<DOT_HIGHEST>(k1, colop(sDAq, 1), qt[1]);
        mma16<DOT_HIGHEST>(k2, colop(sDA, 1), bkt[1]);
        drain(k1, k2);
      } else if (nb == 2) {
        mma16<DOT_HIGHEST>(k1, colop(sDAq, 0), qt[0]);
        mma16<DOT_HIGHEST>(k2, colop(sDA, 0), bkt[0]);
        mma16<DOT_HIGHEST>(k1, colop(sDAq, 1), qt[1]);
        mma16<DOT_HIGHEST>(k2, colop(sDA, 1), bkt[1]);
        drain(k1, k2);
      } else {
        mma16<DOT_HIGHEST>(k1, colop(sDAq, 0), qt[0]);
        mma16<DOT_HIGHEST>(k2, colop(sDA, 0), bkt[0]);
        drain(k1, k2);
      }
      const float4 cc = cb ? cbl[1] : cbl[0], kk = cb ? kt[1] : kt[0];
      const float cv[4] = {cc.x, cc.y, cc.z, cc.w}, ktv[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        if (St::rtile(wv, m) != tj) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = scale * k1[e] + k2[e];
          dk4[m][e] += x * cv[e];
          dgc4[m][e] -= x * ktv[e];
        }
      }
    }
  };
  if constexpr (STD) {
    constexpr Piece P0{0, 0, 32, 1, 0, 0, 32, 0}, P1{32, 32, 32, 1, 32, 32, 64, 0}, P2{32, 0, 32, 0, 32, 0, 0, 0};
    b4_piece(P0);
    b4_piece(P1);
    b4_piece(P2);
  } else {
    for (int pi = 0; pi < cf.pieces.n; ++pi) {
      const Piece pc = load_piece(cf.pieces.p[pi]);
      if (elementwise(pc)) continue;
      b4_piece(pc);
    }
  }

  // Elementwise pieces: the lean diagonal's (b4.py:20-30) with the exact
  // E = exp(clip(gc_i - gc_j, +-diff_clip)), the others with E = row leg x column leg (the
  // factorised form above, one element at a time).  In both, dE/dgc_i = E = -dE/dgc_j.
  if constexpr (ELEM) {
    for (int pi = 0; pi < cf.pieces.n; ++pi) {
      const Piece pc = load_piece(cf.pieces.p[pi]);
      if (!elementwise(pc)) continue;
      const bool exact = EM == EM_LEAN || (lean && pc.kind != 0);
      const float dc = cf.diff_clip;
#pragma unroll
      for (int m = 0; m < NTW; ++m) {
        const int rt = St::rtile(wv, m);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int x = 16 * rt + 4 * g + e;      // row (as i) or column (as j) of the piece
          const float gx = sG[x * LD + dcol];
          if (x >= pc.row0 && x < pc.row0 + pc.P) {
            float sq = 0.f, sbk = 0.f;
            const float rl = exact ? 0.f : piece_row_leg(pc, sG, LD, x, dcol, ar, az);
            for (int jl = 0; jl < pc.P; ++jl) {
              const int j = pc.col0 + jl;
              const float E = exact ? expf(clip_nan(gx - sG[j * LD + dcol], -dc, dc))
                                    : rl * piece_col_leg(pc, sG, LD, j, dcol, ar, az);
              const float ek = E * k[j * D + dcol];
              sq += sDAq[x * LT + j] * ek;
              sbk += sDA[x * LT + j] * ek;
            }
            const float xs = scale * sq, qx = q[x * D + dcol], bkx = b[x * D + dcol] * k[x * D + dcol];
            dq4[m][e] += xs;
            dbk4[m][e] += sbk;
            dgc4[m][e] += qx * xs + bkx * sbk;
          }
          if (x >= pc.col0 && x < pc.col0 + pc.P) {
            float s2 = 0.f;
            const float cl = exact ? 0.f : piece_col_leg(pc, sG, LD, x, dcol, ar, az);
            for (int il = 0; il < pc.P; ++il) {
              const int i = pc.row0 + il;
              const float E = exact ? expf(clip_nan(sG[i * LD + dcol] - gx, -dc, dc))
                                    : piece_row_leg(pc, sG, LD, i, dcol, ar, az) * cl;
              const float M = sDAq[i * LT + x] * (scale * q[i * D + dcol]) + sDA[i * LT + x] * (b[i * D + dcol] * k[i * D + dcol]);
              s2 += M * E;
            }
            dk4[m][e] += s2;
            dgc4[m][e] -= k[x * D + dcol] * s2;
          }
        }
      }
    }
  }

  // PERSIST: the next chunk's DMA has had B4 to land; it is waited for here (the compiler
  // does not know of it) and published by the barrier that ends the chunk.  A and g of a chunk
  // are loaded into registers at its start (held across the loop they would spill).
  if constexpr (PERSIST) __builtin_amdgcn_s_waitcnt(WAIT_VMCNT0);

  // per owned tile: dkb = A^T dWp (mega.py:42; A^T is upper triangular, so row tile rt only
  // sees k blocks >= rt), then the gate gradients (mega.py:45-51) and the
  // combine with B4 (mega.py:52-59).  Row T-1 also needs the last-row decay term (mega.py:50),
  // a sum over all rows: its dgc is finished after the loop.
  // With RT_STATIC (D = 128) a wave owns whole columns: the gradient tiles are stored from the
  // accumulator layout (four rows of 64 contiguous bytes per instruction), and the column sum
  // and B5 stay inside the wave, so no barrier follows P4.  Otherwise two waves share a
  // column: the tiles leave through a per-wave 16x16 LDS transpose (in the dAqk buffer, free
  // once every wave has left B4), dgc goes to X1 and B5 runs over the workgroup.  Every
  // gradient store is a streaming (non-temporal) one: no load is issued after them in this
  // chunk, and written lines that skip the cache drain faster before the next chunk's loads
  // (measured: 143 -> 128 us in one probe pair).
  float* __restrict__ o_dq = a.dq + tio;
  float* __restrict__ o_dk = a.dk + tio;
  float* __restrict__ o_db = a.db + tio;
  float* sDgc = sX1;
  const float gl = sG[(T - 1) * LD + dcol];
  const float dlast = owned(3) && g == 3 ? a.dlast[(size_t)chunk * D + dcol] : 0.f;
  float part = 0.f, fix3 = 0.f, fix4 = 0.f;
  float dgv[NTW][4];                                 // RT_STATIC: this lane's dgc3 + dgc4
  if constexpr (B3 != DOT_HIGHEST) gate_loads();
  static_assert(NW * 16 * TRP <= T * LT, "transpose tiles fit in the dAqk buffer");
  if constexpr (!RT_STATIC) __syncthreads();
  float* tr = sDAq + wv * 16 * TRP;
#pragma unroll
  for (int m = 0; m < NTW; ++m) {
    const int rt = St::rtile(wv, m), i0 = 16 * rt + 4 * g;
    const float4 dqg4 = dqg4s[m], dkg4 = dkg4s[m];
    f4 dkb = {0.f, 0.f, 0.f, 0.f};
    // straight-line MFMA chain: skip the zero k blocks only where rt is a compile-time value
    auto acol = [&](int kb) {
      const float* ac = sA + (16 * kb + 4 * g) * LT + 16 * rt + r;
      return make_float4(ac[0], ac[LT], ac[2 * LT], ac[3 * LT]);
    };
    if constexpr (B3 == DOT_HIGHEST) {
#pragma unroll
      for (int kb = RT_STATIC ? m : 0; kb < 4; ++kb) mma16<B3>(dkb, acol(kb), dwpc[kb]);
    } else {
      mma_chain<B3, 4>(dkb, RT_STATIC ? m : 0, acol, [&](int kb) { return dwpc[kb]; });
    }
    drain(dkb);
    const float4 q4 = pick4(qv, rt), k4 = pick4(kv, rt), b4 = pick4(bv, rt);
    const float qa[4] = {q4.x, q4.y, q4.z, q4.w}, ka[4] = {k4.x, k4.y, k4.z, k4.w}, ba[4] = {b4.x, b4.y, b4.z, b4.w};
    const float qga[4] = {dqg4.x, dqg4.y, dqg4.z, dqg4.w}, kga[4] = {dkg4.x, dkg4.y, dkg4.z, dkg4.w};
    float oq[4], ok[4], ob[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = i0 + e;
      const float be = ba[e], ke = ka[e], qe = qa[e];
      const float gi = sG[i * LD + dcol];
      const float egc = exp_nonpos(gi), ekg = exp_nonpos(gl - gi);
      // derivative masks 1{x <= 0} of exp(min(x, 0)); the reference's 1{x < 0} (bwd/mega.py:47-48)
      // drops the terms of rows whose later gates round away against gc (gl - gc == 0 in fp32)
      const float mgc = gi <= 0.f ? 1.f : 0.f, mkg = (gl - gi) <= 0.f ? 1.f : 0.f;
      const float kbv = (be * ke) * egc;
      const float kg = sanitize(ke * ekg, clip), qg = sanitize(qe * egc, clip);
      const float dqg = qga[e], dkg = kga[e];
      const float dx = dkg * kg;
      part += dx * mkg;
      const float dq3 = dqg * egc;
      const float dk3 = (dkb[e] * egc) * be + dkg * ekg;
      const float db3 = (dkb[e] * egc) * ke;
      const float dgc3 = ((dkb[e] * kbv) * mgc + (dqg * qg) * mgc) - dx * mkg;
      const float dqv = sanitize(dq4[m][e], clip);
      const float dbkv = sanitize(dbk4[m][e], clip);
      const float dk4v = sanitize(dk4[m][e] + dbkv * be, clip);
      const float db4v = sanitize(dbkv * ke, clip);
      const float dgc4v = sanitize(dgc4[m][e], clip);
      oq[e] = sanitize(dq3 + dqv, clip);
      ok[e] = sanitize(dk3 + dk4v, clip);
      ob[e] = sanitize(db3 + db4v, clip);
      if (i == T - 1) {
        fix3 = dgc3;
        fix4 = dgc4v;
      }
      const float dgcv = sanitize(dgc3, clip) + dgc4v;
      if constexpr (RT_STATIC) dgv[m][e] = dgcv;
      else if (i != T - 1) sDgc[i * LD + dcol] = dgcv;
    }
    if constexpr (RT_STATIC) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        __builtin_nontemporal_store(oq[e], o_dq + (i0 + e) * D + dcol);
        __builtin_nontemporal_store(ok[e], o_dk + (i0 + e) * D + dcol);
        __builtin_nontemporal_store(ob[e], o_db + (i0 + e) * D + dcol);
      }
    } else {
      // lane (r, g) after the transpose: row 16 rt + r, columns 16 strip + 4 g .. + 3
      const int ro = (16 * rt + r) * D + 16 * strip + 4 * g;
      stg4(o_dq + ro, wave_transpose16(tr, make_float4(oq[0], oq[1], oq[2], oq[3]), r, g));
      stg4(o_dk + ro, wave_transpose16(tr, make_float4(ok[0], ok[1], ok[2], ok[3]), r, g));
      stg4(o_db + ro, wave_transpose16(tr, make_float4(ob[0], ob[1], ob[2], ob[3]), r, g));
    }
  }
  // last-row decay gradient: sum over all rows of the column (lanes g, then the waves of the
  // strip in order) + e^gamma sum_v(dh_next h_pre) [gl <= 0]
  part += __shfl_xor(part, 16);
  part += __shfl_xor(part, 32);
  if constexpr (RT_STATIC) {
    // the strip is this wave's alone; row T-1 is element 3 of row tile 3 on the lanes g = 3
    const float dec = exp_nonpos(gl), mdec = gl <= 0.f ? 1.f : 0.f;
    const float colsum = part + dec * dlast * mdec;
    if (g == 3) dgv[NTW - 1][3] = sanitize(fix3 + colsum, clip) + fix4;
    // B5 (mega.py:53): dg = reverse cumsum over the chunk rows, row order (t, g, e): within a
    // lane over e, then the later lane groups g of the same row tile (exclusive suffix across
    // lanes r + 16 g), then the totals of the later row tiles.
    float* __restrict__ o_dg = a.dg + tio;
    float later = 0.f;                               // sum of the row tiles below t
#pragma unroll
    for (int t = NTW - 1; t >= 0; --t) {
      float x[4];
      x[3] = dgv[t][3];
#pragma unroll
      for (int e = 2; e >= 0; --e) x[e] = x[e + 1] + dgv[t][e];
      const float s = x[0];
      const float s1 = __shfl(s, (l + 16) & 63), s2 = __shfl(s, (l + 32) & 63), s3 = __shfl(s, (l + 48) & 63);
      const float suf = ((g < 3 ? s1 : 0.f) + (g < 2 ? s2 : 0.f)) + (g < 1 ? s3 : 0.f);
      const float tot = __shfl(suf + s, r);          // lane g = 0: the row tile's total
      const float off = later + suf;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __builtin_nontemporal_store(sanitize(x[e] + off, clip), o_dg + (16 * t + 4 * g + e) * D + dcol);
      later += tot;
    }
    // every wave is done with sA before the next chunk's A is written there
    if constexpr (PERSIST) __syncthreads();
    continue;
  }
  if (g == 0) sColP[wv * 16 + r] = part;
  __syncthreads();
  if (owned(3) && g == 3) {
    float colsum = 0.f;
    for (int w2 = strip; w2 < NW; w2 += St::NS) colsum += sColP[w2 * 16 + r];
    const float dec = exp_nonpos(gl), mdec = gl <= 0.f ? 1.f : 0.f;
    colsum += dec * dlast * mdec;
    sDgc[(T - 1) * LD + dcol] = sanitize(fix3 + colsum, clip) + fix4;
  }
  __syncthreads();

  // B5: dg = reverse cumsum over the chunk rows of dgc3 + dgc4 (mega.py:53).  Thread t owns
  // float4 column t % (D/4) over a run of RUN rows; runs below are added in order.
  {
    constexpr int NQ = D / 4, NSEG = NT / NQ, RUN = T / NSEG;
    const int d = 4 * (tid % NQ), sg = tid / NQ;
    float4 x[RUN];
#pragma unroll
    for (int i = 0; i < RUN; ++i) x[i] = ld4(sDgc + (sg * RUN + i) * LD + d);
#pragma unroll
    for (int i = RUN - 2; i >= 0; --i) x[i] = add4(x[i + 1], x[i]);
    float* sTot = sDA;                             // dAkk is no longer needed
    st4(sTot + sg * LD + d, x[0]);                 // run totals
    __syncthreads();
    float4 off = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s2 = NSEG - 1; s2 > sg; --s2) off = add4(off, ld4(sTot + s2 * LD + d));
#pragma unroll
    for (int i = 0; i < RUN; ++i) stg4(a.dg + tio + (sg * RUN + i) * D + d, san4(add4(x[i], off), clip));
  }
  }
}

// ------------------------------------------------------------------------------------
// bwd_pre: the reverse scan's dO terms for one chunk (mega.py:34-35), which do not depend on dh:
//   X = Aqk^T dO (T x D),  Y = Qg^T (s dO) (D x D)
// as MFMA tiles whose accumulators are exactly the fragment blocks the scan loads: tile
// (tp, vb) of X is block (vb, tp) of FA(X^T), tile (kb, vb) of Y is block (vb, kb) of FA(Y^T).
// A operands: blocks of Aqk^T / Qg^T, i.e. blocks of FA(Aqk) / FA(Qg) (the forward's
// residual) turned around by a per-wave LDS transpose; the B operand (dO columns) from LDS.
// ------------------------------------------------------------------------------------
template <int D, int B3>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdPreArgs a) {
  constexpr int LT = T + 4, NT = 256, NW = NT / WAVE, NVB = D / 16, NKB = D / 16, NYW = NKB / NW;
  __shared__ __attribute__((aligned(16))) float sOT[D * LT];      // dO^T: [value][token]
  const int chunk = blockIdx.x, tid = threadIdx.x, w = wave_id(), l = lane_id(), r = l & 15, g = l >> 4;
  const size_t tb = (size_t)chunk * T * D, sb = (size_t)chunk * T * T, hb = (size_t)chunk * D * D;
  const float* __restrict__ dout = a.dout + io_off<D>(a.cfg, chunk);
  // A operands, once per wave: X row block tp = w (all four k blocks: the blocks u < tp of
  // Aqk^T are exact zeros), Y row blocks kb = w + NW m.  Block (w, u) of Aqk^T in the operand
  // layout is block (u, w) of Aqk in the accumulator layout: FA(Aqk) block (u, w) transposed.
  // The transpose tiles lie in sOT, which is filled after a barrier.
  static_assert(NW * 16 * TRP <= D * LT, "transpose tiles fit in the dO^T buffer");
  float* tr = sOT + w * 16 * TRP;
  float4 ax[4], ay[NYW][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ax[u] = ldg4(a.aqk_f + sb + frag_blk(u, w, T) + 4 * l);
#pragma unroll
    for (int m = 0; m < NYW; ++m) ay[m][u] = ldg4(a.qg_f + tb + frag_blk(u, w + NW * m, D) + 4 * l);
  }
  // dO in the same memory round trip (row-major items, scattered into dO^T below)
  constexpr int NDO = T * D / 4 / NT;
  float4 xo[NDO];
#pragma unroll
  for (int it = 0; it < NDO; ++it) xo[it] = ld4(dout + 4 * (tid + it * NT));
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    ax[u] = wave_transpose16(tr, ax[u], r, g);
#pragma unroll
    for (int m = 0; m < NYW; ++m) ay[m][u] = wave_transpose16(tr, ay[m][u], r, g);
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < NDO; ++it) {
    const int f = tid + it * NT, t = f / (D / 4), c = 4 * (f % (D / 4));
    const float4 x = xo[it];
    sOT[(c + 0) * LT + t] = x.x;
    sOT[(c + 1) * LT + t] = x.y;
    sOT[(c + 2) * LT + t] = x.z;
    sOT[(c + 3) * LT + t] = x.w;
  }
  __syncthreads();
  const float scale = a.cfg.scale;
#pragma unroll 1
  for (int vb = 0; vb < NVB; ++vb) {
    // B operand: dO[16u + 4g + e][16 vb + r] = dO^T[16 vb + r][16u + 4g + e]; and s dO
    float4 bo[4], bs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      bo[u] = ld4(sOT + (16 * vb + r) * LT + 16 * u + 4 * g);
      bs[u] = scale4(bo[u], scale);
    }
    f4 accx = {0.f, 0.f, 0.f, 0.f};
    mma_chain<B3, 4>(accx, 0, [&](int u) { return ax[u]; }, [&](int u) { return bo[u]; });
    f4 accy[NYW];
#pragma unroll
    for (int m = 0; m < NYW; ++m) {
      accy[m] = f4{0.f, 0.f, 0.f, 0.f};
      mma_chain<B3, 4>(accy[m], 0, [&](int u) { return ay[m][u]; }, [&](int u) { return bs[u]; });
    }
    drain(accx);
    stg4(a.x_f + tb + frag_blk(vb, w, T) + 4 * l, f4_to_float4(accx));
#pragma unroll
    for (int m = 0; m < NYW; ++m) {
      drain(accy[m]);
      stg4(a.y_f + hb + frag_blk(vb, w + NW * m, D) + 4 * l, f4_to_float4(accy[m]));
    }
  }
}

hipError_t launch_bwd_pre(int D, const BwdPreArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((bwd_pre_kernel<128, M>), dim3(a.n_chunks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((bwd_pre_kernel<64, M>), dim3(a.n_chunks), dim3(256), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_bwd_state(int D, const BwdStateArgs& a, hipStream_t s) {
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    if (D == 128) hipLaunchKernelGGL((bwd_state_kernel<128, M>), dim3(a.n_chunks), dim3(8 * WAVE), 0, s, a);
    else hipLaunchKernelGGL((bwd_state_kernel<64, M>), dim3(a.n_chunks), dim3(4 * WAVE), 0, s, a);
    return 0;
  });
  return hipGetLastError();
}

hipError_t launch_bwd_state_rc(int D, const BwdStateRcArgs& a, hipStream_t s) {
  const int nblk = CkptBlocks(a.nc, a.ckpt, a.cfg.group).nblk;
  dispatch_mode(a.cfg.b3_mode, [&](auto m3) {
    dispatch_mode(a.cfg.dot_mode, [&](auto md) {
      constexpr int M3 = decltype(m3)::value, MD = decltype(md)::value;
      if (D == 128)
        hipLaunchKernelGGL((bwd_state_rc_kernel<128, 4, M3, MD>), dim3(a.n_bh * nblk * 2), dim3(4 * WAVE), 0, s, a);
      else
        hipLaunchKernelGGL((bwd_state_rc_kernel<64, 4, M3, MD>), dim3(a.n_bh * nblk), dim3(4 * WAVE), 0, s, a);
      return 0;
    });
    return 0;
  });
  return hipGetLastError();
}

// The piece list of the standard geometry (make_pieces(64, 64, 32)): the two 32 x 32 diagonal
// blocks and the level-2 block below the first.
static bool std_pieces(const PieceList& pl) {
  const int ref[3][7] = {{0, 0, 32, 1, 0, 0, 32}, {32, 32, 32, 1, 32, 32, 64}, {32, 0, 32, 0, 32, 0, 0}};
  if (pl.n != 3) return false;
  for (int i = 0; i < 3; ++i) {
    const Piece& p = pl.p[i];
    const int got[7] = {p.row0, p.col0, p.P, p.kind, p.anchor, p.s0, p.s1};
    for (int j = 0; j < 7; ++j)
      if (got[j] != ref[i][j]) return false;
  }
  return true;
}

hipError_t launch_bwd_wy(int D, const BwdWyArgs& a, hipStream_t s) {
  // elementwise pieces: pieces of side 8 (every piece has side min(bs2, 32)), or the lean diagonal
  const bool mix = a.cfg.pieces.p[0].P < 16, elem = mix || a.cfg.diag == DIAG_LEAN;
  const bool std_geom = !elem && std_pieces(a.cfg.pieces);
  // kind-2 pieces on the factorised path read the anchor buffer
  if (!elem && a.cfg.pieces.p[0].kind == 2 && !a.anc) return hipErrorInvalidValue;
  // D = 128 BTL kernels are persistent: one workgroup per CU (their LDS admits no second).
  dim3 pgrid;
  const hipError_t e = persistent_grid(a.n_chunks, &pgrid);
  if (e != hipSuccess) return e;
  dispatch_mode(a.cfg.b3_mode, [&](auto m) {
    constexpr int M = decltype(m)::value;
    const dim3 grid(a.n_chunks), block(512);
    if (D == 128) {
      if (mix) hipLaunchKernelGGL((bwd_wy_kernel<128, M, false, EM_MIX>), grid, block, 0, s, a);
      else if (elem) hipLaunchKernelGGL((bwd_wy_kernel<128, M, false, EM_LEAN>), grid, block, 0, s, a);
      else if (std_geom) hipLaunchKernelGGL((bwd_wy_kernel<128, M, true, EM_NONE>), pgrid, block, 0, s, a);
      else hipLaunchKernelGGL((bwd_wy_kernel<128, M, false, EM_NONE>), pgrid, block, 0, s, a);
    } else {
      if (mix) hipLaunchKernelGGL((bwd_wy_kernel<64, M, false, EM_MIX>), grid, block, 0, s, a);
      else if (elem) hipLaunchKernelGGL((bwd_wy_kernel<64, M, false, EM_LEAN>), grid, block, 0, s, a);
      else if (std_geom) hipLaunchKernelGGL((bwd_wy_kernel<64, M, true, EM_NONE>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((bwd_wy_kernel<64, M, false, EM_NONE>), grid, block, 0, s, a);
    }
    return 0;
  });
  return hipGetLastError();
}

}  // namespace gdn2
