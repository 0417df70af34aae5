// The elementwise work on either side of the gated DeltaNet op, fused into single passes:
//
//  * gated RMSNorm of the op's output (fla's FusedRMSNormGated in GatedDeltaNet; the reference's
//    self.norm(y) * silu(g), archbench/layers/nsgdn.py:539-541), per row of DV channels (one head of one token):
//      y = x * rsqrt(mean(x^2) + eps) * w * silu(gate)            (gate optional)
//    forward and backward (dx, dgate, dw), fp32 arithmetic, x / gate / y in the activation dtype;
//  * L2 normalisation of q and k per head with a scale (nsgdn.py:527-528, F.normalize(.) * DK^-1/2; fla's
//    use_qk_l2norm_in_kernel):  y = scale * x / max(||x||, eps), forward and backward on the same kernels;
//  * the gate functions (nsgdn.py:531-533; fla GatedDeltaNet's g and beta):
//      g    = max(-exp(A_log[h]) * softplus(a + dt_bias[h]), g_min)
//      beta = beta_scale * sigmoid(b + b_bias[h])
//    forward and backward (da, db, dA_log, ddt_bias, db_bias).
//
// Rows of the norm: x, y, dy, dx, dgate [rows, DV] contiguous; w [DV] fp32; gate rows either contiguous too or
// read in place from a wider tensor: lines of gpl rows (gpl * DV contiguous channels, e.g. the heads of one
// token) ldg elements apart, row r at (r / gpl) * ldg + (r % gpl) * DV (gate_row below).  Each lane holds 8 consecutive
// channels (one 16-byte bf16 access), a row spans DV/8 lanes and its sums run on DPP; a wave takes 64/(DV/8)
// rows per access group and NORM_U groups per batch of loads.  HBM-bound: forward reads x and gate and writes y;
// the backward reads x, gate and dy and writes dx and dgate.  dw is summed per workgroup in a fixed order and the
// workgroup partials by column_sum_kernel (deterministic).
#include <math.h>

#include <algorithm>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int NORM_U = 4;      // row groups per load batch
constexpr int NORM_WAVES = 4;  // waves per workgroup

// what a row pass computes
enum NormMode { RMS = 0, RMS_GATE = 1, L2 = 2 };

// element offset of gate row r (gpl = 1: r * ldg; the host keeps rows below 2^32 otherwise)
template <int DV>
__device__ __forceinline__ int64_t gate_row(int64_t r, int64_t ldg, int gpl) {
  if (gpl == 1) return r * ldg;
  const uint32_t line = (uint32_t)r / (uint32_t)gpl;
  return (int64_t)line * ldg + (int64_t)((uint32_t)r - line * (uint32_t)gpl) * DV;
}

template <typename T, int DV, int MODE>
__global__ __launch_bounds__(64 * NORM_WAVES) void row_norm_fwd_kernel(const T* __restrict__ x,
                                                                       const T* __restrict__ gate,
                                                                       const float* __restrict__ w,
                                                                       T* __restrict__ y, int64_t rows, float eps,
                                                                       float scale, int64_t ldg, int gpl) {
  constexpr int LPR = DV / 8, RPW = 64 / LPR, U = NORM_U;
  constexpr bool GATE = MODE == RMS_GATE;
  const int l = lane_id();
  const int sub = l / LPR, c0 = (l % LPR) * 8;
  const int64_t row0 = ((int64_t)blockIdx.x * NORM_WAVES + wave_id()) * (RPW * U);
  if (row0 >= rows) return;  // waves never synchronise
  float wk[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wk[j] = MODE == L2 ? scale : (w ? w[c0 + j] : 1.f);
  Row8<T> xr[U], gr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = min(row0 + u * RPW + sub, rows - 1);  // clamped: rows past the end are loaded, not stored
    xr[u].load(x + r * DV + c0);
    if constexpr (GATE) gr[u].load(gate + gate_row<DV>(r, ldg, gpl) + c0);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = row0 + u * RPW + sub;
    float xs[8], o[8];
    xr[u].get(xs);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += xs[j] * xs[j];
    const float rs = MODE == L2 ? 1.f / fmaxf(sqrtf(lane_group_sum<LPR>(ss)), eps)
                                : rsqrtf(lane_group_sum<LPR>(ss) * (1.f / DV) + eps);
    if constexpr (GATE) {
      float gs[8];
      gr[u].get(gs);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = xs[j] * rs * wk[j] * (gs[j] * fast_sigmoid(gs[j]));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = xs[j] * rs * wk[j];
    }
    if (r < rows) store_row8(y + r * DV + c0, o);
  }
}

// Persistent over batches of NORM_U row groups (wave v takes batches v, v + waves, ...); dw accumulates in
// registers, then over the rows of a wave (lane shuffles) and the waves of the workgroup (LDS, fixed order) into
// one partial row per workgroup.
template <typename T, int DV, int MODE>
__global__ __launch_bounds__(64 * NORM_WAVES) void row_norm_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ gate, const float* __restrict__ w, const T* __restrict__ dy,
    T* __restrict__ dx, T* __restrict__ dgate, float* __restrict__ dw_part, int64_t rows, float eps, float scale,
    int64_t ldg, int gpl) {
  constexpr int LPR = DV / 8, RPW = 64 / LPR, U = NORM_U;
  constexpr bool GATE = MODE == RMS_GATE;
  __shared__ float red[NORM_WAVES][DV];
  const int l = lane_id(), wv = wave_id();
  const int sub = l / LPR, c0 = (l % LPR) * 8;
  float wk[8], dwa[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    wk[j] = MODE == L2 ? scale : (w ? w[c0 + j] : 1.f);
    dwa[j] = 0.f;
  }
  const int64_t stride = (int64_t)gridDim.x * NORM_WAVES * (RPW * U);
  for (int64_t row0 = ((int64_t)blockIdx.x * NORM_WAVES + wv) * (RPW * U); row0 < rows; row0 += stride) {
    Row8<T> xr[U], gr[U], dr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = min(row0 + u * RPW + sub, rows - 1);
      xr[u].load(x + r * DV + c0);
      dr[u].load(dy + r * DV + c0);
      if constexpr (GATE) gr[u].load(gate + gate_row<DV>(r, ldg, gpl) + c0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = row0 + u * RPW + sub;
      const bool ok = r < rows;
      float xs[8], ds[8], gs[8], sg[8];
      xr[u].get(xs);
      dr[u].get(ds);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += xs[j] * xs[j];
      // RMS: rs = (mean(x^2) + eps)^-1/2, smooth in x.  L2: rs = 1 / max(||x||, eps), constant (no row term in
      // the gradient) while the norm is below eps
      const float nrm2 = lane_group_sum<LPR>(ss);
      const float rs = MODE == L2 ? 1.f / fmaxf(sqrtf(nrm2), eps) : rsqrtf(nrm2 * (1.f / DV) + eps);
      const float rowterm = MODE == L2 ? (sqrtf(nrm2) > eps ? 1.f : 0.f) : 1.f / DV;
      float xh[8], du[8], dot = 0.f;
      if constexpr (GATE) gr[u].get(gs);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xh[j] = xs[j] * rs;
        float dyh = ds[j];
        if constexpr (GATE) {
          sg[j] = fast_sigmoid(gs[j]);
          dyh *= gs[j] * sg[j];
        }
        dwa[j] += ok ? dyh * xh[j] : 0.f;
        du[j] = dyh * wk[j];
        dot += du[j] * xh[j];
      }
      dot = lane_group_sum<LPR>(dot) * rowterm;
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = rs * (du[j] - xh[j] * dot);
      if (ok) store_row8(dx + r * DV + c0, o);
      if constexpr (GATE) {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = ds[j] * xh[j] * wk[j] * sg[j] * (1.f + gs[j] * (1.f - sg[j]));
        if (ok) store_row8(dgate + r * DV + c0, o);
      }
    }
  }
  if constexpr (MODE == L2) return;  // no parameter gradient (uniform exit: no barrier follows)
  // lanes with the same channels (l mod LPR) hold different rows: butterfly over them
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (LPR <= 8) dwa[j] = xor8_sum(dwa[j]);
    if constexpr (LPR <= 16) dwa[j] = xor16_sum(dwa[j]);
    dwa[j] = xor32_sum(dwa[j]);
  }
  if (sub == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) red[wv][c0 + j] = dwa[j];
  }
  __syncthreads();
  for (int c = threadIdx.x; c < DV; c += 64 * NORM_WAVES) {
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < NORM_WAVES; ++v) s += red[v][c];
    dw_part[(int64_t)blockIdx.x * DV + c] = s;
  }
}

// ------------------------------------------------------------------------------------------------ gates
__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }  // torch threshold

template <typename T>
__global__ __launch_bounds__(256) void gates_fwd_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                        const float* __restrict__ A_log,
                                                        const float* __restrict__ dt_bias,
                                                        const float* __restrict__ b_bias, float* __restrict__ g,
                                                        float* __restrict__ beta, int64_t n, int H, int64_t lda,
                                                        float beta_scale, float g_min) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t t = e / H;
    const int h = (int)(e - t * H);
    const float xa = to_f(a[t * lda + h]) + (dt_bias ? dt_bias[h] : 0.f);
    g[e] = fmaxf(-expf(A_log[h]) * softplus_f(xa), g_min);
    const float xb = to_f(b[t * lda + h]) + (b_bias ? b_bias[h] : 0.f);
    beta[e] = beta_scale * (1.f / (1.f + expf(-xb)));
  }
}

constexpr int GATE_TILE = 1024;  // elements per workgroup tile of the backward (TN tokens x H heads)

// One workgroup per TN = max(1, GATE_TILE / H) tokens: per-element gradients go to da, db and to LDS, then thread
// c < 3H sums column c of the tile in token order -> one partial row [dA_log (H) | ddt_bias (H) | db_bias (H)].
template <typename T>
__global__ __launch_bounds__(256) void gates_bwd_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                        const float* __restrict__ A_log,
                                                        const float* __restrict__ dt_bias,
                                                        const float* __restrict__ b_bias,
                                                        const float* __restrict__ dg, const float* __restrict__ dbeta,
                                                        T* __restrict__ da, T* __restrict__ db,
                                                        float* __restrict__ part, int64_t ntok, int H, int TN,
                                                        int64_t lda, int64_t ldd, float beta_scale, float g_min) {
  __shared__ float sA[GATE_TILE], sX[GATE_TILE], sY[GATE_TILE];
  const int64_t tok0 = (int64_t)blockIdx.x * TN;
  const int ntile = (int)min((int64_t)TN, ntok - tok0) * H;
  const int64_t e0 = tok0 * H;
  for (int i = threadIdx.x; i < ntile; i += 256) {
    const int64_t e = e0 + i;
    const int tl = i / H, h = i - tl * H;
    const int64_t ia = (tok0 + tl) * lda + h, id = (tok0 + tl) * ldd + h;  // a, b and da, db rows lda, ldd apart
    const float xa = to_f(a[ia]) + (dt_bias ? dt_bias[h] : 0.f);
    const float eA = expf(A_log[h]);
    const float gu = -eA * softplus_f(xa);  // before the clamp
    const float dgu = gu >= g_min ? dg[e] : 0.f;  // clamp_min passes the gradient where the input is >= g_min
    const float dxa = dgu * -eA * (xa > 20.f ? 1.f : 1.f / (1.f + expf(-xa)));
    const float xb = to_f(b[ia]) + (b_bias ? b_bias[h] : 0.f);
    const float s = 1.f / (1.f + expf(-xb));
    const float dxb = dbeta[e] * beta_scale * s * (1.f - s);
    da[id] = from_f<T>(dxa);
    db[id] = from_f<T>(dxb);
    sA[i] = dgu * gu;  // d/dA_log of -exp(A_log) softplus(.) is the value itself
    sX[i] = dxa;
    sY[i] = dxb;
  }
  __syncthreads();
  const int nt = ntile / H;
  for (int c = threadIdx.x; c < 3 * H; c += 256) {
    const float* src = c < H ? sA : (c < 2 * H ? sX : sY);
    const int h = c % H;
    float s = 0.f;
    for (int t = 0; t < nt; ++t) s += src[t * H + h];
    part[(int64_t)blockIdx.x * 3 * H + c] = s;
  }
}

// ----------------------------------------------------------------------------------------------- launchers
static int norm_grid_fwd(int64_t rows, int DV) {
  const int64_t per_wg = (int64_t)(64 / (DV / 8)) * NORM_U * NORM_WAVES;
  return (int)((rows + per_wg - 1) / per_wg);
}

int norm_bwd_workgroups(int64_t rows, int DV) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(norm_grid_fwd(rows, DV), 3 * (int64_t)device_cu_count()));
}

size_t norm_ws_bytes(int64_t rows, int DV) {
  return ((size_t)norm_bwd_workgroups(rows, DV) * DV * 4 + 255) & ~size_t(255);
}

bool norm_shape_supported(int DV) { return DV == 64 || DV == 128 || DV == 256; }

template <typename T, int DV, int MODE>
static hipError_t norm_k(const NormArgs& a, bool backward) {
  if (!backward) {
    row_norm_fwd_kernel<T, DV, MODE><<<dim3(norm_grid_fwd(a.rows, DV)), 64 * NORM_WAVES, 0, a.stream>>>(
        static_cast<const T*>(a.x), static_cast<const T*>(a.gate), a.w, static_cast<T*>(a.y), a.rows, a.eps,
        a.scale, a.ldg ? a.ldg : DV, a.ldg ? a.gpl : 1);
    return hipGetLastError();
  }
  const int nwg = norm_bwd_workgroups(a.rows, DV);
  float* part = static_cast<float*>(a.ws);
  row_norm_bwd_kernel<T, DV, MODE><<<dim3(nwg), 64 * NORM_WAVES, 0, a.stream>>>(
      static_cast<const T*>(a.x), static_cast<const T*>(a.gate), a.w, static_cast<const T*>(a.dy),
      static_cast<T*>(a.dx), static_cast<T*>(a.dgate), part, a.rows, a.eps, a.scale, a.ldg ? a.ldg : DV,
      a.ldg ? a.gpl : 1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || MODE == L2 || !a.dw) return e;
  return launch_column_sum(part, nwg, DV, ColumnOut{{a.dw, nullptr, nullptr}, {DV, 0, 0}}, a.stream);
}

template <typename T, int MODE>
static hipError_t norm_dim(const NormArgs& a, bool backward) {
  switch (a.DV) {
    case 64: return norm_k<T, 64, MODE>(a, backward);
    case 128: return norm_k<T, 128, MODE>(a, backward);
    case 256: return norm_k<T, 256, MODE>(a, backward);
  }
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t norm_mode(const NormArgs& a, bool backward) {
  if (a.l2) return norm_dim<T, L2>(a, backward);
  return a.gate ? norm_dim<T, RMS_GATE>(a, backward) : norm_dim<T, RMS>(a, backward);
}

hipError_t launch_norm(const NormArgs& a, bool backward) {
  return a.dtype == DT_BF16 ? norm_mode<bf16>(a, backward) : norm_mode<float>(a, backward);
}

static int gates_tile_tokens(int H) { return std::max(1, GATE_TILE / H); }

int gates_max_heads() { return GATE_TILE; }

size_t gates_ws_bytes(int64_t ntok, int H) {
  const int64_t nwg = (ntok + gates_tile_tokens(H) - 1) / gates_tile_tokens(H);
  return ((size_t)nwg * 3 * H * 4 + 255) & ~size_t(255);
}

template <typename T>
static hipError_t gates_k(const GateArgs& a, bool backward) {
  const int64_t n = a.ntok * a.H;
  if (!backward) {
    const int64_t nb = std::min<int64_t>((n + 255) / 256, 8 * (int64_t)device_cu_count());
    gates_fwd_kernel<T><<<dim3((int)nb), 256, 0, a.stream>>>(static_cast<const T*>(a.a), static_cast<const T*>(a.b),
                                                              a.A_log, a.dt_bias, a.b_bias, a.g, a.beta, n, a.H,
                                                              a.lda ? a.lda : a.H, a.beta_scale, a.g_min);
    return hipGetLastError();
  }
  const int TN = gates_tile_tokens(a.H);
  const int64_t nwg = (a.ntok + TN - 1) / TN;
  float* part = static_cast<float*>(a.ws);
  gates_bwd_kernel<T><<<dim3((int)nwg), 256, 0, a.stream>>>(
      static_cast<const T*>(a.a), static_cast<const T*>(a.b), a.A_log, a.dt_bias, a.b_bias, a.dg, a.dbeta,
      static_cast<T*>(a.da), static_cast<T*>(a.db), part, a.ntok, a.H, TN, a.lda ? a.lda : a.H,
      a.ldd ? a.ldd : a.H, a.beta_scale, a.g_min);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // each partial row is [dA_log (H) | ddt_bias (H) | db_bias (H)]
  return launch_column_sum(part, nwg, 3 * a.H, ColumnOut{{a.dA_log, a.ddt_bias, a.db_bias}, {a.H, a.H, a.H}},
                           a.stream);
}

hipError_t launch_gates(const GateArgs& a, bool backward) {
  return a.dtype == DT_BF16 ? gates_k<bf16>(a, backward) : gates_k<float>(a, backward);
}

}  // namespace gdn
