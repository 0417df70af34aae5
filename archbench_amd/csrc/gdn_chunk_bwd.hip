// Chunkwise gated delta rule, backward.
//
// The backward recomputes the chunk factors (fwd_intra) and the entering state of every chunk (fwd_state in
// backward mode) rather than keeping them from the forward, then runs:
//
// bwd_state: one workgroup per (V block, b*h), reverse over chunks, fp32 dS slab in MFMA accumulators.
//     dR  = P^T dO + Kd dS_C                         Kd = diag(exp(G_C - G)) K
//     dS0 = gamma_C dS_C + s (diag(gamma) Q)^T dO - W^T dR
//   Writes dS_C (the gradient w.r.t. the state leaving each chunk) and dR per chunk, and dh0.
//   (The reverse state-gradient recurrence of fla's chunk_gated_delta_rule_bwd_dhu, called at
//   archbench/layers/nsgdn.py:378.)
//
// bwd_intra: one workgroup per (chunk, b*h) with the full K and V of the chunk; all gradients:
//     dq  = s gamma (dO S0^T) + (dP o sE) K                         dP = dO R^T  (i >= j)
//     dk  = dte (R dS_C^T) + (dP o sE)^T Q + beta gamma (Tm^T dW) + (D + D^T) K
//     dv  = beta (Tm^T dR)                                          dW = -dR S0^T
//     dA  = -Tm^T (dW X^T + dR Y^T) Tm^T  (strict lower),  D = dA o beta_i E,  X = beta gamma K, Y = beta V
//     dbeta = gamma (Tm^T dW . k) + (Tm^T dR . v) + rowsum(dA o KK o E)
//     dG  = s gamma (dO S0^T . q) - dte (R dS_C^T . k) + beta gamma (Tm^T dW . k)
//           + rowsum - colsum of (dP o P + dA o A),   dG_last += sum dte (R dS_C^T . k) + gamma_C <dS_C, S0>
//     dg  = reverse chunk-local cumsum of dG
//   (fla's chunk_bwd_dv_local + chunk_bwd_dqkwg, the WY backward of nsgdn.py:279-330 and the reverse cumsum
//   of nsgdn.py:381, fused per chunk.)  Reductions are deterministic: no atomics anywhere.
#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

template <typename T, int K, int BV>
__global__ __launch_bounds__(NTHR) void bwd_state_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ dout, const float* __restrict__ dhT,
    float* __restrict__ dh0, const T* __restrict__ wsP, const T* __restrict__ wsW, const float* __restrict__ wsGc,
    T* __restrict__ wsdH, T* __restrict__ wsdR, int T_, int H, int V, int NT, float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT;
  constexpr int NCT = BV / 16;
  constexpr int NST = (K / 16) * NCT;
  constexpr int SPW = NST / NWAVE;
  static_assert(NST % NWAVE == 0, "state slab must split evenly over the waves");
  __shared__ __attribute__((aligned(16))) T sKd[CH * LK];
  __shared__ __attribute__((aligned(16))) T sQgt[K * LC];
  __shared__ __attribute__((aligned(16))) T sWt[K * LC];
  __shared__ __attribute__((aligned(16))) T sPt[CH * LC];
  __shared__ __attribute__((aligned(16))) T sdOt[BV * LC];
  __shared__ __attribute__((aligned(16))) T sdSt[BV * LK];
  __shared__ __attribute__((aligned(16))) T sdRt[BV * LC];
  __shared__ float sG[CH];

  const int vb = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int v0 = vb * BV;
  const int tid = threadIdx.x, w = wave_id();
  const int64_t sbase = (int64_t)bh * K * V;

  f32x4 dS[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 16 * mi + acc_row(i), vc = 16 * ni + acc_col();
      dS[s][i] = dhT ? dhT[sbase + (int64_t)d * V + v0 + vc] : 0.f;
    }
  }

  for (int c = NT - 1; c >= 0; --c) {
    const int t0 = c * CH;
    const int nvalid = min(CH, T_ - t0);
    const int64_t row0 = ((int64_t)b * T_ + t0) * H + h;
    const int64_t cidx = (int64_t)bh * NT + c;
    if (tid < CH) sG[tid] = wsGc[cidx * CH + tid];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * mi + acc_row(i), vc = 16 * ni + acc_col();
        const T val = from_f<T>(dS[s][i]);
        sdSt[vc * LK + d] = val;
        wsdH[cidx * K * V + (int64_t)d * V + v0 + vc] = val;
      }
    }
    {
      const T* Wc = wsW + cidx * CH * K;
      for (int idx = tid; idx < CH * K; idx += NTHR) {
        const int i = idx / K, d = idx - i * K;
        sWt[d * LC + i] = Wc[idx];
      }
      const T* Pc = wsP + cidx * CH * CH;
      for (int idx = tid; idx < CH * CH; idx += NTHR) {
        const int i = idx >> 6, j = idx & 63;
        sPt[j * LC + i] = Pc[idx];
      }
      for (int idx = tid; idx < CH * BV; idx += NTHR) {
        const int i = idx / BV, n = idx - i * BV;
        sdOt[n * LC + i] = i < nvalid ? dout[(row0 + (int64_t)i * H) * V + v0 + n] : from_f<T>(0.f);
      }
    }
    __syncthreads();
    const float GC = sG[CH - 1];
    for (int idx = tid; idx < CH * K; idx += NTHR) {
      const int j = idx / K, d = idx - j * K;
      const float kv = j < nvalid ? to_f(k[(row0 + (int64_t)j * H) * K + d]) : 0.f;
      const float qv = j < nvalid ? to_f(q[(row0 + (int64_t)j * H) * K + d]) : 0.f;
      sKd[j * LK + d] = from_f<T>(__expf(GC - sG[j]) * kv);
      sQgt[d * LC + j] = from_f<T>(__expf(sG[j]) * qv);
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NCT; ++n) {
      f32x4 dr = {0.f, 0.f, 0.f, 0.f};
      mma_blk<true, true, CH>(dr, sPt, LC, 16 * w, sdOt, LC, 16 * n);
      mma_blk<true, true, K>(dr, sKd, LK, 16 * w, sdSt, LK, 16 * n);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * w + acc_row(i), vc = 16 * n + acc_col();
        const T val = from_f<T>(dr[i]);
        sdRt[vc * LC + r] = val;
        wsdR[(cidx * CH + r) * V + v0 + vc] = val;
      }
    }
    __syncthreads();
    const float gC = __expf(GC);
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
      f32x4 a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
      mma_blk<true, true, CH>(a1, sQgt, LC, 16 * mi, sdOt, LC, 16 * ni);
      mma_blk<true, true, CH>(a2, sWt, LC, 16 * mi, sdRt, LC, 16 * ni);
      dS[s] = gC * dS[s] + scale * a1 - a2;
    }
    __syncthreads();
  }
  if (dh0) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * mi + acc_row(i), vc = 16 * ni + acc_col();
        dh0[sbase + (int64_t)d * V + v0 + vc] = dS[s][i];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Sum of the 4 rows a lane holds plus the other 3 lane groups: the per-column sum of a 16x16 tile.
__device__ __forceinline__ float colsum_tile(const f32x4& x) {
  float s = x[0] + x[1] + x[2] + x[3];
  s += __shfl_xor(s, 16);
  s += __shfl_xor(s, 32);
  return s;
}

template <typename T, int K, int V, int VS>
__global__ __launch_bounds__(NTHR) void bwd_intra_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const float* __restrict__ beta,
    const T* __restrict__ dout, const T* __restrict__ wsTm, const float* __restrict__ wsGc,
    const T* __restrict__ wsH, const T* __restrict__ wsR, const T* __restrict__ wsdH, const T* __restrict__ wsdR,
    T* __restrict__ dq, T* __restrict__ dk, T* __restrict__ dv, float* __restrict__ dg,
    float* __restrict__ dbeta, int T_, int H, int NT, float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LS = VS + PT;
  constexpr int NKT = K / 16;   // column tiles over K
  constexpr int NVT = VS / 16;  // column tiles over a V slab
  // slab region: V phase {dO, R, dR, V : CH x LS; S0, dSC : K x LS}; K phase {dWn : CH x LK; dTm, M1, D, dPm : CH x LC}
  constexpr int SLAB_V = 4 * CH * LS + 2 * K * LS;
  constexpr int SLAB_K = CH * LK + 4 * CH * LC;
  constexpr int SLAB = SLAB_V > SLAB_K ? SLAB_V : SLAB_K;
  __shared__ __attribute__((aligned(16))) T sQ[CH * LK];
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];
  __shared__ __attribute__((aligned(16))) T sTm[CH * LC];
  __shared__ __attribute__((aligned(16))) T slab[SLAB];
  __shared__ float sG[CH], sB[CH], sdG[CH], sLast[CH], sColZ[NWAVE][CH], sRed[NWAVE];

  T* sdO = slab;
  T* sR = sdO + CH * LS;
  T* sdR = sR + CH * LS;
  T* sV = sdR + CH * LS;
  T* sS0 = sV + CH * LS;
  T* sdSC = sS0 + K * LS;

  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * CH;
  const int nvalid = min(CH, T_ - t0);
  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int64_t row0 = ((int64_t)b * T_ + t0) * H + h;
  const int64_t cidx = (int64_t)bh * NT + c;

  g2s_rows(sQ, LK, q + row0 * K, (int64_t)H * K, CH, K, nvalid);
  g2s_rows(sK, LK, k + row0 * K, (int64_t)H * K, CH, K, nvalid);
  g2s_rows(sTm, LC, wsTm + cidx * CH * CH, (int64_t)CH, CH, CH, CH);
  if (tid < CH) {
    sG[tid] = wsGc[cidx * CH + tid];
    sB[tid] = tid < nvalid ? beta[row0 + (int64_t)tid * H] : 0.f;
  }

  // ---- V phase: contractions over V, slab by slab -------------------------------------------------------
  f32x4 aP[4], aTV[4], aQg[NKT], aKd[NKT], aWn[NKT];
#pragma unroll
  for (int n = 0; n < 4; ++n) aP[n] = aTV[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int n = 0; n < NKT; ++n) aQg[n] = aKd[n] = aWn[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float dbV[4] = {0.f, 0.f, 0.f, 0.f};
  float sdot = 0.f;  // partial <dS_C, S0>

  for (int vs = 0; vs < V; vs += VS) {
    g2s_rows(sdO, LS, dout + row0 * V + vs, (int64_t)H * V, CH, VS, nvalid);
    g2s_rows(sV, LS, v + row0 * V + vs, (int64_t)H * V, CH, VS, nvalid);
    g2s_rows(sR, LS, wsR + cidx * CH * V + vs, (int64_t)V, CH, VS, CH);
    g2s_rows(sdR, LS, wsdR + cidx * CH * V + vs, (int64_t)V, CH, VS, CH);
    g2s_rows(sS0, LS, wsH + cidx * K * V + vs, (int64_t)V, K, VS, K);
    g2s_rows(sdSC, LS, wsdH + cidx * K * V + vs, (int64_t)V, K, VS, K);
    __syncthreads();
    for (int idx = tid; idx < K * VS; idx += NTHR) {
      const int d = idx / VS, n = idx - d * VS;
      sdot += to_f(sdSC[d * LS + n]) * to_f(sS0[d * LS + n]);
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      mma_blk<true, true, VS>(aP[n], sdO, LS, 16 * w, sR, LS, 16 * n);
      mma_blk<true, true, VS>(aTV[n], sdR, LS, 16 * w, sV, LS, 16 * n);
    }
#pragma unroll
    for (int n = 0; n < NKT; ++n) {
      mma_blk<true, true, VS>(aQg[n], sdO, LS, 16 * w, sS0, LS, 16 * n);
      mma_blk<true, true, VS>(aKd[n], sR, LS, 16 * w, sdSC, LS, 16 * n);
      mma_blk<true, true, VS>(aWn[n], sdR, LS, 16 * w, sS0, LS, 16 * n);
    }
    // dY = Tm^T dR for this slab: dv = beta dY, dbeta += dY . v
#pragma unroll
    for (int n = 0; n < NVT; ++n) {
      f32x4 dy = {0.f, 0.f, 0.f, 0.f};
      mma_blk<false, false, CH>(dy, sTm, LC, 16 * w, sdR, LS, 16 * n);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * w + acc_row(i), vc = 16 * n + acc_col();
        dbV[i] += dy[i] * to_f(sV[r * LS + vc]);
        if (r < nvalid) dv[(row0 + (int64_t)r * H) * V + vs + vc] = from_f<T>(sB[r] * dy[i]);
      }
    }
    __syncthreads();
  }
  // block reduce <dS_C, S0>
  {
    float x = sdot;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    if (l == 0) sRed[w] = x;
  }

  // ---- K phase --------------------------------------------------------------------------------------------
  T* sdWn = slab;                 // CH x LK   dR S0^T (= -dW)
  T* sdTm = sdWn + CH * LK;       // CH x LC
  T* sM1 = sdTm + CH * LC;        // CH x LC   dTm Tm^T
  T* sD = sM1 + CH * LC;          // CH x LC   D = dA o beta_i E
  T* sdPm = sD + CH * LC;         // CH x LC   dP o s E

  const int lg = l >> 4;  // lane group: rows 4*lg .. 4*lg+3 of each tile
  float gam[4], dte[4], bet[4];
  const float GC = sG[CH - 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * w + acc_row(i);
    gam[i] = __expf(sG[r]);
    dte[i] = __expf(GC - sG[r]);
    bet[i] = sB[r];
  }
  // row dots from the V-phase accumulators
  float rq[4] = {0.f, 0.f, 0.f, 0.f}, rk[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int n = 0; n < NKT; ++n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i), d = 16 * n + acc_col();
      rq[i] += aQg[n][i] * to_f(sQ[r * LK + d]);
      rk[i] += aKd[n][i] * to_f(sK[r * LK + d]);
      sdWn[r * LK + d] = from_f<T>(aWn[n][i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rq[i] = sum16(rq[i]);
    rk[i] = sum16(rk[i]);
    dbV[i] = sum16(dbV[i]);
  }
  __syncthreads();

  // dX = Tm^T dW = -Tm^T dWn (rows of this wave), and rx = dX . k
  f32x4 aX[NKT];
  float rx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int n = 0; n < NKT; ++n) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    mma_blk<false, false, CH>(t, sTm, LC, 16 * w, sdWn, LK, 16 * n);
    aX[n] = -t;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i), d = 16 * n + acc_col();
      rx[i] += aX[n][i] * to_f(sK[r * LK + d]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) rx[i] = sum16(rx[i]);
  // dTm rows:  dTm_ij = -beta_j gamma_j (dWn K^T)_ij + beta_j (dR V^T)_ij
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    mma_blk<true, true, K>(t, sdWn, LK, 16 * w, sK, LK, 16 * n);
    const int cc = 16 * n + acc_col();
    const float bj = sB[cc], gj = __expf(sG[cc]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i);
      sdTm[r * LC + cc] = from_f<T>(-bj * gj * t[i] + bj * aTV[n][i]);
    }
  }
  __syncthreads();
  // M1 = dTm Tm^T (rows of this wave)
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    mma_blk<true, true, CH>(t, sdTm, LC, 16 * w, sTm, LC, 16 * n);
#pragma unroll
    for (int i = 0; i < 4; ++i) sM1[(16 * w + acc_row(i)) * LC + 16 * n + acc_col()] = from_f<T>(t[i]);
  }
  __syncthreads();
  // dA = -Tm^T M1, strict lower; with KK and QK recomputed: D, dPm, dbeta_A and the dG row/col sums
  float rz[4] = {0.f, 0.f, 0.f, 0.f}, dbA[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    f32x4 da = {0.f, 0.f, 0.f, 0.f}, kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
    mma_blk<false, false, CH>(da, sTm, LC, 16 * w, sM1, LC, 16 * n);
    mma_blk<true, true, K>(kk, sK, LK, 16 * w, sK, LK, 16 * n);
    mma_blk<true, true, K>(qk, sQ, LK, 16 * w, sK, LK, 16 * n);
    f32x4 z;
    const int cc = 16 * n + acc_col();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i);
      const float e = (r >= cc) ? __expf(sG[r] - sG[cc]) : 0.f;
      const float dA = (r > cc) ? -da[i] : 0.f;
      const float Aval = bet[i] * kk[i] * e;
      const float dP = (r >= cc) ? aP[n][i] : 0.f;
      const float Pval = scale * e * qk[i];
      sD[r * LC + cc] = from_f<T>(dA * bet[i] * e);
      sdPm[r * LC + cc] = from_f<T>(dP * scale * e);
      dbA[i] += dA * kk[i] * e;
      z[i] = dP * Pval + dA * Aval;
      rz[i] += z[i];
    }
    const float cs = colsum_tile(z);
    if (lg == 0) sColZ[w][cc] = cs;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rz[i] = sum16(rz[i]);
    dbA[i] = sum16(dbA[i]);
  }
  __syncthreads();
  // dq = s gamma dQg + dPm K
#pragma unroll
  for (int n = 0; n < NKT; ++n) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    mma_blk<true, false, CH>(t, sdPm, LC, 16 * w, sK, LK, 16 * n);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i), d = 16 * n + acc_col();
      if (r < nvalid) dq[(row0 + (int64_t)r * H) * K + d] = from_f<T>(scale * gam[i] * aQg[n][i] + t[i]);
    }
  }
  // dk = dte dKd + dPm^T Q + beta gamma dX + D K + D^T K
#pragma unroll
  for (int n = 0; n < NKT; ++n) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    mma_blk<false, false, CH>(t, sdPm, LC, 16 * w, sQ, LK, 16 * n);
    mma_blk<true, false, CH>(t, sD, LC, 16 * w, sK, LK, 16 * n);
    mma_blk<false, false, CH>(t, sD, LC, 16 * w, sK, LK, 16 * n);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i), d = 16 * n + acc_col();
      if (r < nvalid)
        dk[(row0 + (int64_t)r * H) * K + d] =
            from_f<T>(dte[i] * aKd[n][i] + t[i] + bet[i] * gam[i] * aX[n][i]);
    }
  }
  // dbeta and the per-row part of dG (one lane per row)
  if ((l & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i);
      const float db = gam[i] * rx[i] + dbV[i] + dbA[i];
      if (r < nvalid) dbeta[row0 + (int64_t)r * H] = db;
      sdG[r] = scale * gam[i] * rq[i] - dte[i] * rk[i] + bet[i] * gam[i] * rx[i] + rz[i];
      sLast[r] = dte[i] * rk[i];
    }
  }
  __syncthreads();
  if (w == 0) {
    // dG_r -= colsum_r;  dG_last += sum_r dte_r rk_r + gamma_C <dS_C, S0>;  dg = reverse cumsum of dG
    float x = sdG[l] - (sColZ[0][l] + sColZ[1][l] + sColZ[2][l] + sColZ[3][l]);
    float last = sLast[l];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) last += __shfl_xor(last, off);
    last += __expf(GC) * (sRed[0] + sRed[1] + sRed[2] + sRed[3]);
    if (l == CH - 1) x += last;
    const float incl = wave_inclusive_scan(x);
    const float total = __shfl(incl, 63);
    if (l < nvalid) dg[row0 + (int64_t)l * H] = total - incl + x;
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T> constexpr int state_bv_b() { return 32; }

template <typename T, int K>
static hipError_t bwd_state_k(const ChunkArgs& a) {
  constexpr int BV = state_bv_b<T>();
  dim3 grid(a.V / BV, a.B * a.H);
  bwd_state_kernel<T, K, BV><<<grid, NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.dout), a.dhT, a.dh0,
      static_cast<const T*>(a.ws.P), static_cast<const T*>(a.ws.W), a.ws.Gc, static_cast<T*>(a.ws.dhs),
      static_cast<T*>(a.ws.dRs), a.T, a.H, a.V, a.NT, a.scale);
  return hipGetLastError();
}

template <typename T, int K, int V>
static hipError_t bwd_intra_kv(const ChunkArgs& a) {
  constexpr int VS = sizeof(T) == 2 ? 64 : 32;
  dim3 grid(a.NT, a.B * a.H);
  bwd_intra_kernel<T, K, V, VS><<<grid, NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.v), a.beta,
      static_cast<const T*>(a.dout), static_cast<const T*>(a.ws.Tm), a.ws.Gc, static_cast<const T*>(a.ws.hs),
      static_cast<const T*>(a.ws.Rs), static_cast<const T*>(a.ws.dhs), static_cast<const T*>(a.ws.dRs),
      static_cast<T*>(a.dq), static_cast<T*>(a.dk), static_cast<T*>(a.dv), a.dg, a.dbeta, a.T, a.H, a.NT,
      a.scale);
  return hipGetLastError();
}

template <typename T, int K>
static hipError_t bwd_intra_k(const ChunkArgs& a) {
  if (a.V == 64) return bwd_intra_kv<T, K, 64>(a);
  if (a.V == 128) return bwd_intra_kv<T, K, 128>(a);
  if (a.V == 256) return bwd_intra_kv<T, K, 256>(a);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_state(const ChunkArgs& a) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return bwd_state_k<bf16, 64>(a);
    if (a.K == 128) return bwd_state_k<bf16, 128>(a);
  } else {
    if (a.K == 64) return bwd_state_k<float, 64>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_intra(const ChunkArgs& a) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return bwd_intra_k<bf16, 64>(a);
    if (a.K == 128) return bwd_intra_k<bf16, 128>(a);
  } else {
    if (a.K == 64) return bwd_intra_k<float, 64>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace gdn
