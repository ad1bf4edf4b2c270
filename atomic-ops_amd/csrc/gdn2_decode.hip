// Token recurrence of the GDN-2 operator for serving, on gfx950: the single-token decode step
// and the tail of the forward-only prefill (the tokens after its last full chunk), with the
// semantics of the reference's inference module (notebooks/gdn2_v031_stage2_tpu.ipynb, cell 1,
// INFERENCE_V031: _decode_body and decode_step; the per-token math is reference/ref.py:116-130).
// Per token, for every (batch, head):
//   S = reset ? 0 : state;   h = diag(e^{min(g,0)}) S;   erase_j = sum_d (b k)_d h[d][j];
//   v_new = w v - erase;     h += k v_new^T;              o_j = sum_d h[d][j] (s q)_d;
//   with a cap:  h *= min(1, tau / max(||h||_F, 1e-12))  (per head, NaN propagates);
//   h and o: NaN / +-Inf -> 0;  o stored in the output dtype, the state carried in the state
//   dtype (rounded after every token, as consecutive decode_step calls store it).
// Layout: the value columns of the state are independent, so a workgroup takes a slice of CW
// columns of one (batch, head): CW = 32 (D/32 workgroups per head) without the cap, CW = D with
// it (the cap needs the whole head's norm).  Thread t owns 4 consecutive columns
// (j0 = 4 (t % (CW/4))) and the D/KG key rows of group kg = t / (CW/4), KG = 16, of the state,
// in registers for all tokens of the call: one 16-byte (fp32) or 8-byte (bf16) access per key
// row, the state read from HBM once at the start and written once at the end.  The per-token key
// vectors (s q, k, b k, e^{min(g,0)}) go through LDS (one entry per key row, read by every
// thread of the key group), and each key-direction sum is a per-thread sum over its rows in
// ascending order followed by the KG key groups in the order 0..KG-1 (three barriers per
// token).  The work is element-wise and memory-bound (no MFMA): 2 D^2 state elements per
// (batch, head) and call, plus 7 D per token.
#include "gdn2_kernels.hpp"

namespace gdn2 {

// jnp.nan_to_num(x, nan=0, posinf=0, neginf=0)
__device__ __forceinline__ float finite_or_zero(float x) { return __builtin_isfinite(x) ? x : 0.f; }
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = WAVE / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m);
  return x;
}
// jax.nn.softplus(x) = logaddexp(x, 0) = max(x, 0) + log1p(exp(-|x|)); NaN propagates
__device__ __forceinline__ float softplus(float x) {
  return __builtin_elementwise_maximum(x, 0.f) + log1pf(expf(-fabsf(x)));
}
__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

template <bool BF>
__device__ __forceinline__ float4 ld_quad(const void* p, size_t i) {
  if constexpr (BF) {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    return make_float4(bf16_val(u.x & 0xffffu), bf16_val(u.x >> 16), bf16_val(u.y & 0xffffu), bf16_val(u.y >> 16));
  } else {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
  }
}
template <bool BF>
__device__ __forceinline__ void st_quad(void* p, size_t i, const float4& x) {
  if constexpr (BF) {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = make_uint2(bf16_pack(x.x, x.y), bf16_pack(x.z, x.w));
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = x;
  }
}
template <bool BF>
__device__ __forceinline__ float ld_one(const void* p, size_t i) {
  if constexpr (BF) return bf16_val(static_cast<const uint16_t*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}
__device__ __forceinline__ float4 clean4(const float4& x, bool bf) {
  float4 y = make_float4(finite_or_zero(x.x), finite_or_zero(x.y), finite_or_zero(x.z), finite_or_zero(x.w));
  if (bf) y = make_float4(bf16_round(y.x), bf16_round(y.y), bf16_round(y.z), bf16_round(y.w));
  return y;
}

template <int D, int CW, bool CAP, bool IBF, bool SBF>
__global__ __launch_bounds__(CW / 4 * 16) void decode_kernel(DecodeArgs a) {
  constexpr int KG = 16, NQ = CW / 4, NT = NQ * KG, KPK = D / KG, NS = D / CW, NWV = (NT + WAVE - 1) / WAVE;
  static_assert(NT >= D, "the key vectors are formed by one thread per key row");
  __shared__ float4 sVec[D];          // per token, key row d: (s q_d, k_d, b_d k_d, e^{min(g_d,0)})
  __shared__ float4 sEr[KG][NQ];      // key-group partial sums of the erase term, per column quad
  __shared__ float4 sOut[KG][NQ];     // key-group partial sums of the output
  __shared__ float sNrm[NWV];         // per-wave sums of h^2 (cap)
  const int tid = threadIdx.x, cq = tid % NQ, kg = tid / NQ, d0 = kg * KPK;
  const int bh = blockIdx.x / NS, j0 = (blockIdx.x % NS) * CW + 4 * cq;
  const int bi = bh / a.H, hi = bh - bi * a.H;
  const int l = lane_id(), wv = tid / WAVE;
  const size_t sb = (size_t)bh * D * D;

  float4 h[KPK];
#pragma unroll
  for (int i = 0; i < KPK; ++i)
    h[i] = a.state_in ? ld_quad<SBF>(a.state_in, sb + (size_t)(d0 + i) * D + j0) : make_float4(0.f, 0.f, 0.f, 0.f);

  for (int t = 0; t < a.n_tok; ++t) {
    const size_t io = ((size_t)bh * a.seq_ld + t) * D;
    // this thread's columns of w and v, issued with the key vectors' loads (one round trip)
    float4 wj = ld_quad<IBF>(a.w, io + j0);
    const float4 vj = ld_quad<IBF>(a.v, io + j0);
    if (a.reset && a.reset[(size_t)bi * a.n_tok + t]) {
#pragma unroll
      for (int i = 0; i < KPK; ++i) h[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // the token's key vectors (threads 0 .. D-1, whole waves)
    if (tid < D) {
      float qd = ld_one<IBF>(a.q, io + tid), kd = ld_one<IBF>(a.k, io + tid);
      float bd = ld_one<IBF>(a.b, io + tid), gd = ld_one<IBF>(a.g, io + tid);
      if (a.fuse) {
        // the prologue of _decode_body (fuse_prologue): every wave forms the full l2 sums itself
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int m = l; m < D; m += WAVE) {
          const float x = ld_one<IBF>(a.q, io + m), y = ld_one<IBF>(a.k, io + m);
          sq = fmaf(x, x, sq);
          sk = fmaf(y, y, sk);
        }
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        qd *= 1.f / sqrtf(sq + 1e-6f);
        kd *= 1.f / sqrtf(sk + 1e-6f);
        bd = sigmoid(bd);
        gd = -expf(a.a_log[hi]) * softplus(gd + a.dt_bias[tid]);
      }
      sVec[tid] = make_float4(a.scale * qd, kd, bd * kd, exp_nonpos(gd));
    }
    __syncthreads();
    float4 ep = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < KPK; ++i) {
      const float4 x = sVec[d0 + i];
      h[i] = scale4(h[i], x.w);
      ep = make_float4(fmaf(x.z, h[i].x, ep.x), fmaf(x.z, h[i].y, ep.y), fmaf(x.z, h[i].z, ep.z), fmaf(x.z, h[i].w, ep.w));
    }
    sEr[kg][cq] = ep;
    __syncthreads();
    float4 er = sEr[0][cq];
#pragma unroll
    for (int m = 1; m < KG; ++m) er = add4(er, sEr[m][cq]);
    if (a.fuse) wj = make_float4(sigmoid(wj.x), sigmoid(wj.y), sigmoid(wj.z), sigmoid(wj.w));
    const float4 vn = make_float4(wj.x * vj.x - er.x, wj.y * vj.y - er.y, wj.z * vj.z - er.z, wj.w * vj.w - er.w);
    float4 op = make_float4(0.f, 0.f, 0.f, 0.f);
    float np = 0.f;
#pragma unroll
    for (int i = 0; i < KPK; ++i) {
      const float4 x = sVec[d0 + i];
      h[i] = make_float4(fmaf(x.y, vn.x, h[i].x), fmaf(x.y, vn.y, h[i].y), fmaf(x.y, vn.z, h[i].z), fmaf(x.y, vn.w, h[i].w));
      op = make_float4(fmaf(h[i].x, x.x, op.x), fmaf(h[i].y, x.x, op.y), fmaf(h[i].z, x.x, op.z), fmaf(h[i].w, x.x, op.w));
      if constexpr (CAP) np = fmaf(h[i].x, h[i].x, fmaf(h[i].y, h[i].y, fmaf(h[i].z, h[i].z, fmaf(h[i].w, h[i].w, np))));
    }
    sOut[kg][cq] = op;
    if constexpr (CAP) {
      np = wave_sum(np);
      if (l == 0) sNrm[wv] = np;
    }
    __syncthreads();
    if (kg == 0) {
      float4 o = sOut[0][cq];
#pragma unroll
      for (int m = 1; m < KG; ++m) o = add4(o, sOut[m][cq]);
      o = clean4(o, false);
      if (a.out_bf16) st_quad<true>(a.o, io + j0, o);
      else st_quad<false>(a.o, io + j0, o);
    }
    if constexpr (CAP) {
      float n2 = 0.f;
#pragma unroll
      for (int m = 0; m < NWV; ++m) n2 += sNrm[m];
      const float nrm = sqrtf(n2);
      const float f = __builtin_elementwise_minimum(1.f, a.tau / __builtin_elementwise_maximum(nrm, 1e-12f));
#pragma unroll
      for (int i = 0; i < KPK; ++i) h[i] = scale4(h[i], f);
    }
#pragma unroll
    for (int i = 0; i < KPK; ++i) h[i] = clean4(h[i], SBF);
  }
#pragma unroll
  for (int i = 0; i < KPK; ++i) st_quad<SBF>(a.state_out, sb + (size_t)(d0 + i) * D + j0, h[i]);
}

template <int D, bool CAP, bool IBF, bool SBF>
void launch_decode_t(const DecodeArgs& a, int n_bh, hipStream_t s) {
  constexpr int CW = CAP ? D : 32;
  hipLaunchKernelGGL((decode_kernel<D, CW, CAP, IBF, SBF>), dim3(n_bh * (D / CW)), dim3(CW / 4 * 16), 0, s, a);
}

template <int D, bool CAP>
void launch_decode_d(const DecodeArgs& a, int n_bh, hipStream_t s) {
  if (a.in_bf16) {
    if (a.state_bf16) launch_decode_t<D, CAP, true, true>(a, n_bh, s);
    else launch_decode_t<D, CAP, true, false>(a, n_bh, s);
  } else {
    if (a.state_bf16) launch_decode_t<D, CAP, false, true>(a, n_bh, s);
    else launch_decode_t<D, CAP, false, false>(a, n_bh, s);
  }
}

hipError_t launch_decode(int D, const DecodeArgs& a, int n_bh, hipStream_t s) {
  if (D == 128) {
    if (a.cap) launch_decode_d<128, true>(a, n_bh, s);
    else launch_decode_d<128, false>(a, n_bh, s);
  } else {
    if (a.cap) launch_decode_d<64, true>(a, n_bh, s);
    else launch_decode_d<64, false>(a, n_bh, s);
  }
  return hipGetLastError();
}

}  // namespace gdn2
