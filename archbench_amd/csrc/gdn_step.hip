// Single-token recurrent decode step of the gated delta rule, state updated in place.
//
// Per (b, h), with the fp32 state S [K, V] (row-major, V contiguous), alpha = exp(g), scale s:
//     r = beta (v - alpha S^T k),   S <- alpha S + k r^T,   o = S_new^T (s q) = alpha S^T (s q) + r (k . s q)
// (the per-token body of archbench/layers/nsgdn.py:413-416 with u = beta k, nsgdn.py:69).
//
// HBM-bound: S is read once and written once.  One workgroup owns one (b, h) state; thread (rg, cg) holds
// rows [rg*RPT, rg*RPT + RPT) of the float4 column group cg in registers between the two passes, so the
// column reductions S^T k and S^T q come from the same read that feeds the update.  Consecutive lanes own
// consecutive float4 columns, so every load and store is a full coalesced row segment.
#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

template <typename T, int K, int V>
__global__ __launch_bounds__(256) void step_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ v, const float* __restrict__ g,
                                                   const float* __restrict__ beta, float* __restrict__ state,
                                                   T* __restrict__ o, float scale) {
  constexpr int CG = V / 4;      // float4 column groups
  constexpr int RG = 256 / CG;   // row groups
  constexpr int RPT = K / RG;    // rows per thread
  static_assert(RG * CG == 256 && RPT * RG == K, "unsupported step shape");
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int cg = tid % CG, rg = tid / CG;

  __shared__ float sk[K], sq[K];
  __shared__ f32x4 red_k[RG][CG], red_q[RG][CG];
  __shared__ float s_kq;

  f32x4* Sp = reinterpret_cast<f32x4*>(state + (int64_t)bh * K * V);
  f32x4 S[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) S[r] = __builtin_nontemporal_load(Sp + (rg * RPT + r) * CG + cg);
  for (int i = tid; i < K; i += 256) {
    sk[i] = to_f(k[(int64_t)bh * K + i]);
    sq[i] = to_f(q[(int64_t)bh * K + i]) * scale;
  }
  __syncthreads();
  if (tid < 64) {
    float x = 0.f;
    for (int i = tid; i < K; i += 64) x += sk[i] * sq[i];
    x = wave_sum64(x);
    if (tid == 0) s_kq = x;
  }
  f32x4 ak = {0.f, 0.f, 0.f, 0.f}, aq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const float kr = sk[rg * RPT + r], qr = sq[rg * RPT + r];
    ak += S[r] * kr;
    aq += S[r] * qr;
  }
  red_k[rg][cg] = ak;
  red_q[rg][cg] = aq;
  __syncthreads();
  f32x4 tk = red_k[0][cg], tq = red_q[0][cg];
#pragma unroll
  for (int i = 1; i < RG; ++i) {
    tk += red_k[i][cg];
    tq += red_q[i][cg];
  }
  const float a = __expf(g[bh]);
  const float b = beta[bh];
  const float kq = s_kq;
  f32x4 vv;
#pragma unroll
  for (int j = 0; j < 4; ++j) vv[j] = to_f(v[(int64_t)bh * V + 4 * cg + j]);
  const f32x4 rr = b * (vv - a * tk);
  if (rg == 0) {
    const f32x4 oo = a * tq + rr * kq;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[(int64_t)bh * V + 4 * cg + j] = from_f<T>(oo[j]);
  }
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const f32x4 x = a * S[r] + sk[rg * RPT + r] * rr;
    __builtin_nontemporal_store(x, Sp + (rg * RPT + r) * CG + cg);
  }
}

template <typename T, int K, int V>
static hipError_t launch_step_kv(const StepArgs& a) {
  step_kernel<T, K, V><<<dim3(a.B * a.H), dim3(256), 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.v), a.g, a.beta, a.state,
      static_cast<T*>(a.o), a.scale);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_step_t(const StepArgs& a) {
  if (a.K == 64 && a.V == 64) return launch_step_kv<T, 64, 64>(a);
  if (a.K == 128 && a.V == 128) return launch_step_kv<T, 128, 128>(a);
  if (a.K == 128 && a.V == 256) return launch_step_kv<T, 128, 256>(a);
  if (a.K == 64 && a.V == 128) return launch_step_kv<T, 64, 128>(a);
  return hipErrorInvalidValue;
}

bool step_shape_supported(int K, int V) {
  return (K == 64 && V == 64) || (K == 128 && V == 128) || (K == 128 && V == 256) || (K == 64 && V == 128);
}

hipError_t launch_step(const StepArgs& a) {
  return a.dtype == DT_BF16 ? launch_step_t<bf16>(a) : launch_step_t<float>(a);
}

}  // namespace gdn
