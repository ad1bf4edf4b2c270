// Token recurrence of the GDN-2 operator for serving, on gfx950: the single-token decode step
// and the tail of the forward-only prefill (the tokens after its last full chunk), with the
// semantics of the reference's inference module (notebooks/gdn2_v031_stage2_tpu.ipynb, cell 1,
// INFERENCE_V031: _decode_body and decode_step; the per-token math is reference/ref.py:118-132).
// Per token, for every (batch, head):
//   S = reset ? 0 : state;   h = diag(e^{min(g,0)}) S;   erase_j = sum_d (b k)_d h[d][j];
//   v_new = w v - erase;     h += k v_new^T;              o_j = sum_d h[d][j] (s q)_d;
//   with a cap:  h *= min(1, tau / max(||h||_F, 1e-12))  (per head, NaN propagates);
//   h and o: NaN / +-Inf -> 0;  o stored in the output dtype, the state carried in the state
//   dtype (rounded after every token, as consecutive decode_step calls store it).
// Layout: one workgroup per (batch, head) with 4 D threads.  Thread t owns value column
// j = t % D and the D/4 key rows of group kg = t / D of the state, in registers for all tokens
// of the call; the state is read from HBM once at the start and written once at the end.  The
// per-token key vectors (s q, k, b k, e^{min(g,0)}) go through LDS (every lane of a wave reads
// the same entry: broadcast), and each key-direction sum is a per-thread sum over its rows in
// ascending order followed by the four key groups in the order 0..3 (three barriers per token).
// The work is element-wise and memory-bound (no MFMA): 2 D^2 state elements per (batch, head)
// and call, plus 7 D per token.
#include "gdn2_kernels.hpp"

namespace gdn2 {

__device__ __forceinline__ float in_at(const void* p, size_t i, int bf16) {
  return bf16 ? bf16_val(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}
__device__ __forceinline__ void out_at(void* p, size_t i, float x, int bf16) {
  if (bf16) static_cast<uint16_t*>(p)[i] = (uint16_t)bf16_bits(x);
  else static_cast<float*>(p)[i] = x;
}
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

template <int D>
__global__ __launch_bounds__(4 * D) void decode_kernel(DecodeArgs a) {
  constexpr int KPT = D / 4, NWV = 4 * D / WAVE;
  __shared__ float4 sVec[D];          // per token, channel d: (s q_d, k_d, b_d k_d, e^{min(g_d,0)})
  __shared__ float sErase[4][D];      // key-group partial sums of the erase term
  __shared__ float sOut[4][D];        // key-group partial sums of the output
  __shared__ float sNrm[NWV];         // per-wave sums of h^2 (cap)
  const int tid = threadIdx.x, j = tid % D, kg = tid / D, d0 = kg * KPT;
  const int bh = blockIdx.x, bi = bh / a.H, hi = bh - bi * a.H;
  const int l = lane_id(), wv = wave_id();
  const size_t sb = (size_t)bh * D * D;

  float h[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    h[i] = a.state_in ? in_at(a.state_in, sb + (size_t)(d0 + i) * D + j, a.state_bf16) : 0.f;

  for (int t = 0; t < a.n_tok; ++t) {
    const size_t io = ((size_t)bh * a.seq_ld + t) * D;
    if (a.reset && a.reset[(size_t)bi * a.n_tok + t]) {
#pragma unroll
      for (int i = 0; i < KPT; ++i) h[i] = 0.f;
    }
    // the token's key vectors (threads 0 .. D-1)
    if (tid < D) {
      float qd = in_at(a.q, io + tid, a.in_bf16), kd = in_at(a.k, io + tid, a.in_bf16);
      float bd = in_at(a.b, io + tid, a.in_bf16), gd = in_at(a.g, io + tid, a.in_bf16);
      if (a.fuse) {
        // the prologue of _decode_body (fuse_prologue): every wave forms the full l2 sums itself
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int m = l; m < D; m += WAVE) {
          const float x = in_at(a.q, io + m, a.in_bf16), y = in_at(a.k, io + m, a.in_bf16);
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
    float ep = 0.f;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const float4 x = sVec[d0 + i];
      h[i] *= x.w;
      ep = fmaf(x.z, h[i], ep);
    }
    sErase[kg][j] = ep;
    __syncthreads();
    const float erase = ((sErase[0][j] + sErase[1][j]) + sErase[2][j]) + sErase[3][j];
    float wj = in_at(a.w, io + j, a.in_bf16);
    if (a.fuse) wj = sigmoid(wj);
    const float vnew = wj * in_at(a.v, io + j, a.in_bf16) - erase;
    float op = 0.f, np = 0.f;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const float4 x = sVec[d0 + i];
      h[i] = fmaf(x.y, vnew, h[i]);
      op = fmaf(h[i], x.x, op);
      np = fmaf(h[i], h[i], np);
    }
    sOut[kg][j] = op;
    if (a.cap) {
      np = wave_sum(np);
      if (l == 0) sNrm[wv] = np;
    }
    __syncthreads();
    if (kg == 0) {
      const float o = ((sOut[0][j] + sOut[1][j]) + sOut[2][j]) + sOut[3][j];
      out_at(a.o, io + j, finite_or_zero(o), a.out_bf16);
    }
    if (a.cap) {
      float n2 = 0.f;
#pragma unroll
      for (int m = 0; m < NWV; ++m) n2 += sNrm[m];
      const float nrm = sqrtf(n2);
      const float f = __builtin_elementwise_minimum(1.f, a.tau / __builtin_elementwise_maximum(nrm, 1e-12f));
#pragma unroll
      for (int i = 0; i < KPT; ++i) h[i] *= f;
    }
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      h[i] = finite_or_zero(h[i]);
      if (a.state_bf16) h[i] = bf16_round(h[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < KPT; ++i) out_at(a.state_out, sb + (size_t)(d0 + i) * D + j, h[i], a.state_bf16);
}

hipError_t launch_decode(int D, const DecodeArgs& a, int n_bh, hipStream_t s) {
  if (D == 128) hipLaunchKernelGGL(decode_kernel<128>, dim3(n_bh), dim3(4 * 128), 0, s, a);
  else hipLaunchKernelGGL(decode_kernel<64>, dim3(n_bh), dim3(4 * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace gdn2
