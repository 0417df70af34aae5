// Write direction of the n-step gated DeltaNet (archbench/layers/nsgdn.py:61-75, called at :535-536): per token
// row of K channels (one head of one token),
//     u_1 = beta k,  u_{i+1} = u_i - lam beta (p . u_i) p_perp   (i < n_steps),  p_perp = p - (p . k) k,
// with p the previous token's key in the same sequence (zero at t = 0; nsgdn.py:535).  Every u_i stays in the
// span of k and p_perp, so with s = p . k, pp = p . p, m = p . p_perp = pp - s^2 the whole recursion is scalar:
//     u_i = beta k - c_i p_perp,   c_1 = 0,   c_{i+1} = c_i + x (y - c_i m),   x = lam beta,  y = beta s,
//     u = (beta + c s) k - c p.
// One pass over k reads each row and its predecessor (two row dot products on DPP) and writes u.  The backward
// runs the recursion in reverse on scalars and writes dk, dbeta and a per-row dlam: row t's own terms
// (a du + ds p) plus the gradient that row t + 1 sends to its p (= k_t), recomputed from row t + 1's inputs, so
// every output is written once, by one lane group, with no atomics.  fp32 arithmetic; k, u, du, dk in the
// activation dtype, beta and lam fp32.
#include <hip/hip_runtime.h>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int WD_WAVES = 4;  // waves per workgroup

// Scalars of one row from its (k, p) dot products: a, b with u = a k + b p, and what the backward needs of the
// recursion.  With rho = 1 - x m the recursion is affine, c_{i+1} = rho c_i + x y, so the reverse-mode sums over
// its n - 1 steps -- g_rho = gc F and g_xy = gc E with F = sum_{i=2..n} rho^(n-i) c_{i-1} and
// E = sum_{i=2..n} rho^(n-i) -- are accumulated in the same forward loop (F <- rho F + c, E <- rho E + 1) that
// builds c_n: any n_steps, no per-step storage.
struct WdRow {
  float s, m, x, y, c, F, E, a, b;
  __device__ __forceinline__ void build(float s_, float pp, float beta, float lam, int n) {
    s = s_;
    m = pp - s * s;
    x = lam * beta;
    y = beta * s;
    const float rho = 1.f - x * m;
    c = 0.f;
    F = 0.f;
    E = 0.f;
    for (int i = 1; i < n; ++i) {  // step c_{i+1} = c_i + x (y - c_i m)
      F = rho * F + c;
      E = rho * E + 1.f;
      c = c + x * (y - c * m);
    }
    a = beta + c * s;
    b = -c;
  }
  // Reverse pass from da = du . k, db = du . p: gradients w.r.t. beta, lam and the row's two dot products
  __device__ __forceinline__ void grad(float da, float db, float beta, float lam, float& dbeta, float& dlam,
                                       float& ds, float& dpp) const {
    const float gc = s * da - db;           // dL/dc_n
    const float grho = gc * F, gxy = gc * E;  // through rho = 1 - x m and the constant term x y
    const float gx = y * gxy - m * grho, gy = x * gxy, gm = -x * grho;
    dlam = gx * beta;
    dbeta = da + gx * lam + gy * s;
    ds = c * da + gy * beta - 2.f * s * gm;
    dpp = gm;
  }
};

// rows (b, t, h) = ((b * T + t) * H + h); LPR = K / 8 lanes per row, 8 channels each
template <typename T, int K>
__global__ __launch_bounds__(64 * WD_WAVES) void write_dir_fwd_kernel(const T* __restrict__ k,
                                                                      const float* __restrict__ beta,
                                                                      const float* __restrict__ lam, T* __restrict__ u,
                                                                      int64_t rows, int T_, int H, int n) {
  constexpr int LPR = K / 8, RPW = 64 / LPR;
  const int l = lane_id();
  const int64_t r = ((int64_t)blockIdx.x * WD_WAVES + wave_id()) * RPW + l / LPR;
  const int c0 = (l % LPR) * 8;
  const int64_t rr = r < rows ? r : rows - 1;  // clamped: lanes past the end compute and store nothing
  const int64_t tok = rr / H;
  const int h = (int)(rr - tok * H), t = (int)(tok % T_);
  float kv[8], pv[8];
  Row8<T> kr, pr;
  kr.load(k + rr * K + c0);
  kr.get(kv);
  pr.load(k + (t > 0 ? rr - H : rr) * K + c0);
  pr.get(pv);
  float sp = 0.f, spp = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pv[j] = t > 0 ? pv[j] : 0.f;
    sp += pv[j] * kv[j];
    spp += pv[j] * pv[j];
  }
  WdRow w;
  w.build(lane_group_sum<LPR>(sp), lane_group_sum<LPR>(spp), beta[rr], lam[h], n);
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = w.a * kv[j] + w.b * pv[j];
  if (r < rows) store_row8(u + rr * K + c0, o);
}

template <typename T, int K>
__global__ __launch_bounds__(64 * WD_WAVES) void write_dir_bwd_kernel(
    const T* __restrict__ k, const float* __restrict__ beta, const float* __restrict__ lam, const T* __restrict__ du,
    T* __restrict__ dk, float* __restrict__ dbeta, float* __restrict__ dlam, int64_t rows, int T_, int H, int n) {
  constexpr int LPR = K / 8, RPW = 64 / LPR;
  const int l = lane_id();
  const int64_t r = ((int64_t)blockIdx.x * WD_WAVES + wave_id()) * RPW + l / LPR;
  const int c0 = (l % LPR) * 8;
  const int64_t rr = r < rows ? r : rows - 1;
  const int64_t tok = rr / H;
  const int h = (int)(rr - tok * H), t = (int)(tok % T_);
  const bool has_next = t + 1 < T_;
  const int64_t rn = has_next ? rr + H : rr;
  const float lm = lam[h];
  float kv[8], pv[8], gv[8], kn[8], gn[8];
  {
    Row8<T> a, b, c, d, e;
    a.load(k + rr * K + c0);
    b.load(k + (t > 0 ? rr - H : rr) * K + c0);
    c.load(du + rr * K + c0);
    d.load(k + rn * K + c0);
    e.load(du + rn * K + c0);
    a.get(kv);
    b.get(pv);
    c.get(gv);
    d.get(kn);
    e.get(gn);
  }
  // this row: p = k_{t-1}
  float s1 = 0.f, s2 = 0.f, s3 = 0.f, s4 = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pv[j] = t > 0 ? pv[j] : 0.f;
    s1 += pv[j] * kv[j];
    s2 += pv[j] * pv[j];
    s3 += gv[j] * kv[j];
    s4 += gv[j] * pv[j];
  }
  const float bt = beta[rr];
  WdRow w;
  w.build(lane_group_sum<LPR>(s1), lane_group_sum<LPR>(s2), bt, lm, n);
  float db_, dl_, ds, dpp;
  w.grad(lane_group_sum<LPR>(s3), lane_group_sum<LPR>(s4), bt, lm, db_, dl_, ds, dpp);
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = w.a * gv[j] + ds * pv[j];
  // the next row's gradient w.r.t. its p, which is this row's k: b' du' + ds' k' + 2 dpp' p'  (p' = k_t)
  {
    float n1 = 0.f, n2 = 0.f, n3 = 0.f, n4 = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      n1 += kv[j] * kn[j];
      n2 += kv[j] * kv[j];
      n3 += gn[j] * kn[j];
      n4 += gn[j] * kv[j];
    }
    const float btn = beta[rn];
    WdRow wn;
    wn.build(lane_group_sum<LPR>(n1), lane_group_sum<LPR>(n2), btn, lm, n);
    float dbn, dln, dsn, dppn;
    wn.grad(lane_group_sum<LPR>(n3), lane_group_sum<LPR>(n4), btn, lm, dbn, dln, dsn, dppn);
    if (has_next) {
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] += wn.b * gn[j] + dsn * kn[j] + 2.f * dppn * kv[j];
    }
  }
  if (r < rows) {
    store_row8(dk + rr * K + c0, o);
    if (l % LPR == 0) {
      dbeta[rr] = db_;
      dlam[rr] = dl_;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
bool write_dir_supported(int K, int n_steps) {
  return (K == 64 || K == 128 || K == 256) && n_steps >= 1;
}

template <typename T, int K>
static hipError_t write_dir_k(const WriteDirArgs& a, bool backward) {
  constexpr int RPW = 64 / (K / 8);
  const int64_t rows = (int64_t)a.B * a.T * a.H;
  const dim3 grid((unsigned)((rows + RPW * WD_WAVES - 1) / (RPW * WD_WAVES)));
  if (!backward) {
    write_dir_fwd_kernel<T, K><<<grid, 64 * WD_WAVES, 0, a.stream>>>(
        static_cast<const T*>(a.k), a.beta, a.lam, static_cast<T*>(a.u), rows, a.T, a.H, a.n_steps);
  } else {
    write_dir_bwd_kernel<T, K><<<grid, 64 * WD_WAVES, 0, a.stream>>>(
        static_cast<const T*>(a.k), a.beta, a.lam, static_cast<const T*>(a.du), static_cast<T*>(a.dk), a.dbeta,
        a.dlam, rows, a.T, a.H, a.n_steps);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t write_dir_dim(const WriteDirArgs& a, bool backward) {
  switch (a.K) {
    case 64: return write_dir_k<T, 64>(a, backward);
    case 128: return write_dir_k<T, 128>(a, backward);
    case 256: return write_dir_k<T, 256>(a, backward);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_write_dir(const WriteDirArgs& a, bool backward) {
  return a.dtype == DT_BF16 ? write_dir_dim<bf16>(a, backward) : write_dir_dim<float>(a, backward);
}

}  // namespace gdn
