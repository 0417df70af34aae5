// Cross-entropy forward and backward in one pass over the logits, in place: the loss part of the chunked
// linear + cross-entropy of archbench/fused_ce.py:20-57 (fla's cross_entropy_fwd followed by cross_entropy_bwd
// with inplace_backward on each logits chunk).  Per row i of logits [N, ld] (bf16 or fp32, V classes):
//     lse_i  = log sum_j exp(x_ij)                       loss_i = lse_i - x_i,t_i      (0 if t_i == ignore_index)
//     x_ij  <- dloss * (exp(x_ij - lse_i) - [j == t_i])  (0 for an ignored row)
// One workgroup of 1024 threads per row keeps the whole row in registers (V <= 65536: each thread holds up to 8
// 16-byte pieces), so the logits are read once and written once; max and sum go through DPP wave reductions and
// LDS across the 16 waves; the exponentials use the hardware v_exp_f32 (two instructions each: a precise expf,
// twice per element, made the kernel VALU-bound at 2.9 TB/s).  HBM-bound.
#include <math.h>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int CE_THREADS = 1024;
constexpr int CE_WAVES = CE_THREADS / 64;


// reduce over the block: every thread gets the result
template <bool MAX>
__device__ __forceinline__ float block_reduce(float x, float* red) {
  x = MAX ? wave_max64(x) : wave_sum64(x);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < CE_WAVES; ++i) r = MAX ? fmaxf(r, red[i]) : r + red[i];
  __syncthreads();  // red is reused by the next reduction
  return r;
}

// The row stays packed in registers (NC pieces of 8 elements per thread) and is converted to fp32 again in each
// pass; an empty asm between the passes keeps the compiler from holding fp32 copies instead.  Rows of at most 28
// packed registers per thread (bf16 rows up to V = 57344, fp32 up to 24576) then fit in 64 VGPRs, so two
// 1024-thread workgroups share a CU and one row's loads overlap the other's arithmetic and stores (18% faster
// than one row per CU at V = 50304 bf16).
template <typename T>
__device__ __forceinline__ void keep_packed(Row8<T>& p) {
  if constexpr (sizeof(T) == 2) {
    asm volatile("" : "+v"(p.r));
  } else {
    asm volatile("" : "+v"(p.a));
    asm volatile("" : "+v"(p.b));
  }
}
template <typename T, int NC>
constexpr int ce_waves_per_eu() { return 2 * NC * (int)sizeof(T) <= 28 ? 8 : 4; }  // packed row registers <= 28

// NC: 16-byte pieces per thread (8 elements each); row length V <= NC * 8 * CE_THREADS
template <typename T, int NC>
__global__ __launch_bounds__(CE_THREADS) __attribute__((amdgpu_waves_per_eu(ce_waves_per_eu<T, NC>(), 8)))
void ce_fwd_bwd_kernel(T* __restrict__ logits, const int64_t* __restrict__ target,
                                                                float* __restrict__ loss, float* __restrict__ lse_out,
                                                                const float* __restrict__ dloss_p, int V, int64_t ld,
                                                                int64_t ignore_index) {
  __shared__ float red[CE_WAVES];
  const int64_t row = blockIdx.x;
  T* x = logits + row * ld;
  const int tid = threadIdx.x;
  const int64_t t = target[row];
  const bool ignored = t == ignore_index;
  const bool bad = !ignored && (t < 0 || t >= V);
  Row8<T> piece[NC];
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j0 = (c * CE_THREADS + tid) * 8;
    if (j0 < V) {  // V % 8 == 0: a piece is wholly inside the row or wholly outside
      piece[c].load(x + j0);
      float v[8];
      piece[c].get(v);
#pragma unroll
      for (int e = 0; e < 8; ++e) m = fmaxf(m, v[e]);
    }
  }
  m = block_reduce<true>(m, red);
#pragma unroll
  for (int c = 0; c < NC; ++c) keep_packed(piece[c]);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j0 = (c * CE_THREADS + tid) * 8;
    if (j0 < V) {
      float v[8];
      piece[c].get(v);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += __expf(v[e] - m);
    }
  }
  s = block_reduce<false>(s, red);
#pragma unroll
  for (int c = 0; c < NC; ++c) keep_packed(piece[c]);
  const float lse = m + logf(s);
  if (tid == 0) {
    const float xt = (!ignored && !bad) ? to_f(x[t]) : 0.f;
    loss[row] = ignored ? 0.f : (bad ? NAN : lse - xt);
    if (lse_out) lse_out[row] = lse;
  }
  __syncthreads();  // the target logit is read before the row is overwritten
  const float dl = ignored ? 0.f : (dloss_p ? *dloss_p : 1.f);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j0 = (c * CE_THREADS + tid) * 8;
    if (j0 < V) {
      float v[8];
      piece[c].get(v);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = dl * (__expf(v[e] - lse) - (j0 + e == t ? 1.f : 0.f));
      store_row8(x + j0, v);
    }
  }
}

bool ce_shape_supported(int V, int64_t ld) { return V > 0 && V % 8 == 0 && ld >= V && ld % 8 == 0 && V <= 65536; }

template <typename T, int NC>
static hipError_t ce_k(const CeArgs& a) {
  ce_fwd_bwd_kernel<T, NC><<<dim3((unsigned)a.N), CE_THREADS, 0, a.stream>>>(
      static_cast<T*>(a.logits), a.target, a.loss, a.lse, a.dloss, a.V, a.ld, a.ignore_index);
  return hipGetLastError();
}

template <typename T>
static hipError_t ce_dispatch(const CeArgs& a) {
  const int nc = (a.V + 8 * CE_THREADS - 1) / (8 * CE_THREADS);
  switch (nc) {
    case 1: return ce_k<T, 1>(a);
    case 2: return ce_k<T, 2>(a);
    case 3: return ce_k<T, 3>(a);
    case 4: return ce_k<T, 4>(a);
    case 5: return ce_k<T, 5>(a);
    case 6: return ce_k<T, 6>(a);
    case 7: return ce_k<T, 7>(a);
    case 8: return ce_k<T, 8>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ce(const CeArgs& a) {
  return a.dtype == DT_BF16 ? ce_dispatch<bf16>(a) : ce_dispatch<float>(a);
}

}  // namespace gdn
