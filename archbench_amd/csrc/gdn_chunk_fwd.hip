// Chunkwise gated delta rule, forward: per-chunk WY factors and the inter-chunk state sweep.
//
// Per 64-token chunk (local i, j; G = chunk-local cumsum of g, gamma = exp(G), scale s):
//     A_ij = beta_i (k_i . k_j) exp(G_i - G_j)   (i > j)         Tm = (I + A)^-1  (unit lower triangular)
//     W    = Tm diag(beta gamma) K                                U  = Tm diag(beta) V
//     R    = U - W S0                                              P_ij = s exp(G_i - G_j) (q_i . k_j)  (i >= j)
//     O    = s diag(gamma) Q S0 + P R                              S_C  = gamma_C S0 + (diag(exp(G_C - G)) K)^T R
// This is the algebra of archbench/layers/nsgdn.py:240-249 (beta folded into the rows, as in fla's GDN chunk
// kernels that nsgdn.py:357-362 calls) with the call sequence cumsum -> WY -> state sweep -> output.
//
// fwd_intra: one workgroup per (chunk, b*h).  Everything here is independent of V, so it runs once per chunk:
//   G (wave scan), K K^T and Q K^T on MFMA, the 64x64 inverse in LDS (16x16 diagonal blocks by forward
//   substitution, off-diagonal blocks by fp32 MFMA merges), W = Tm X on MFMA.  Writes Tm, P, W, G.
// fwd_state: one workgroup per (V block, b*h), sequential over chunks.  The fp32 state slab S[K, BV] lives in
//   MFMA accumulators for the whole sweep; per chunk it computes U, R, O and the state update on MFMA.
//   In backward mode it writes the entering state and R of every chunk instead of O.
#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

// ---------------------------------------------------------------------------------------------------------
// 16x16x16 fp32 products for the triangular inverse (k split as slice j: k = 4*(l >> 4) + j).
template <int LD>
__device__ __forceinline__ void mma16_ss(f32x4& c, const float* L, const float* R) {
  const int l = lane_id();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = L[(l & 15) * LD + 4 * (l >> 4) + j];
    const float b = R[(4 * (l >> 4) + j) * LD + (l & 15)];
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
}
// c += L * Y with Y an accumulator tile (lane holds rows 4*(l>>4)+j of column l&15: exactly the B slices).
template <int LD>
__device__ __forceinline__ void mma16_sa(f32x4& c, const float* L, const f32x4& Y) {
  const int l = lane_id();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = L[(l & 15) * LD + 4 * (l >> 4) + j];
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Y[j], c, 0, 0, 0);
  }
}
template <int LD>
__device__ __forceinline__ void store_neg_tile(float* dst, const f32x4& t) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[(4 * (l >> 4) + i) * LD + (l & 15)] = -t[i];
}

// (I + A)^-1 for a strictly lower 64x64 A (fp32, LDS, stride LD) into Ti (zero-initialised, stride LD).
// Must be called by all threads of the workgroup.
template <int LD>
__device__ __forceinline__ void invert_unit_lower64(const float* A, float* Ti) {
  const int w = wave_id(), l = lane_id();
  if (w == 0) {
    // diagonal 16x16 blocks: lane (blk, c) solves column c of block blk by forward substitution
    const int blk = l >> 4, cc = l & 15;
    const float* Ab = A + 16 * blk * LD + 16 * blk;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = (i == cc) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) acc -= Ab[i * LD + j] * x[j];
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Ti[(16 * blk + i) * LD + 16 * blk + cc] = x[i];
  }
  __syncthreads();
  auto blkp = [](const float* base, int i, int j) { return base + 16 * i * LD + 16 * j; };
  auto blkw = [](float* base, int i, int j) { return base + 16 * i * LD + 16 * j; };
  // T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj, by distance i - j
  if (w < 3) {
    const int j = w, i = w + 1;
    f32x4 y = {0.f, 0.f, 0.f, 0.f}, t = {0.f, 0.f, 0.f, 0.f};
    mma16_ss<LD>(y, blkp(A, i, j), blkp(Ti, j, j));
    mma16_sa<LD>(t, blkp(Ti, i, i), y);
    store_neg_tile<LD>(blkw(Ti, i, j), t);
  }
  __syncthreads();
  if (w < 2) {
    const int j = w, i = w + 2;
    f32x4 y = {0.f, 0.f, 0.f, 0.f}, t = {0.f, 0.f, 0.f, 0.f};
    mma16_ss<LD>(y, blkp(A, i, j), blkp(Ti, j, j));
    mma16_ss<LD>(y, blkp(A, i, j + 1), blkp(Ti, j + 1, j));
    mma16_sa<LD>(t, blkp(Ti, i, i), y);
    store_neg_tile<LD>(blkw(Ti, i, j), t);
  }
  __syncthreads();
  if (w == 0) {
    f32x4 y = {0.f, 0.f, 0.f, 0.f}, t = {0.f, 0.f, 0.f, 0.f};
    mma16_ss<LD>(y, blkp(A, 3, 0), blkp(Ti, 0, 0));
    mma16_ss<LD>(y, blkp(A, 3, 1), blkp(Ti, 1, 0));
    mma16_ss<LD>(y, blkp(A, 3, 2), blkp(Ti, 2, 0));
    mma16_sa<LD>(t, blkp(Ti, 3, 3), y);
    store_neg_tile<LD>(blkw(Ti, 3, 0), t);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------
template <typename T, int K>
__global__ __launch_bounds__(NTHR) void fwd_intra_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                         const float* __restrict__ g,
                                                         const float* __restrict__ beta, T* __restrict__ wsTm,
                                                         T* __restrict__ wsP, T* __restrict__ wsW,
                                                         float* __restrict__ wsGc, int T_, int H, int NT,
                                                         float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LF = CH + 4;
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];
  __shared__ __attribute__((aligned(16))) T sQ[CH * LK];
  __shared__ __attribute__((aligned(16))) T sXt[K * LC];
  __shared__ __attribute__((aligned(16))) T sTm[CH * LC];
  __shared__ __attribute__((aligned(16))) float sA[CH * LF];
  __shared__ __attribute__((aligned(16))) float sT[CH * LF];
  __shared__ float sG[CH], sB[CH];

  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int t0 = c * CH;
  const int nvalid = min(CH, T_ - t0);
  const int tid = threadIdx.x, w = wave_id(), l = lane_id();
  const int64_t row0 = ((int64_t)b * T_ + t0) * H + h;
  const int64_t cidx = (int64_t)bh * NT + c;

  g2s_rows(sK, LK, k + row0 * K, (int64_t)H * K, CH, K, nvalid);
  g2s_rows(sQ, LK, q + row0 * K, (int64_t)H * K, CH, K, nvalid);
  for (int i = tid; i < CH * LF; i += NTHR) sT[i] = 0.f;
  if (w == 0) {
    const float gv = l < nvalid ? g[row0 + (int64_t)l * H] : 0.f;
    const float bv = l < nvalid ? beta[row0 + (int64_t)l * H] : 0.f;
    const float G = wave_inclusive_scan(gv);
    sG[l] = G;
    sB[l] = bv;
    wsGc[cidx * CH + l] = G;
  }
  __syncthreads();

  // X^T (d, j) = beta_j gamma_j k_j[d]
  for (int idx = tid; idx < CH * K; idx += NTHR) {
    const int j = idx / K, d = idx - j * K;
    sXt[d * LC + j] = from_f<T>(sB[j] * __expf(sG[j]) * to_f(sK[j * LK + d]));
  }
  // K K^T and Q K^T, row block w
  {
    T* Pout = wsP + cidx * CH * CH;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
      mma_blk<true, true, K>(kk, sK, LK, 16 * w, sK, LK, 16 * n);
      mma_blk<true, true, K>(qk, sQ, LK, 16 * w, sK, LK, 16 * n);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * w + acc_row(i), cc = 16 * n + acc_col();
        const float e = (r >= cc) ? __expf(sG[r] - sG[cc]) : 0.f;
        sA[r * LF + cc] = (r > cc) ? sB[r] * kk[i] * e : 0.f;
        Pout[r * CH + cc] = from_f<T>(scale * qk[i] * e);
      }
    }
  }
  __syncthreads();
  invert_unit_lower64<LF>(sA, sT);
  {
    T* Tout = wsTm + cidx * CH * CH;
    for (int idx = tid; idx < CH * CH; idx += NTHR) {
      const int r = idx >> 6, cc = idx & 63;
      const T val = from_f<T>(sT[r * LF + cc]);
      sTm[r * LC + cc] = val;
      Tout[idx] = val;
    }
  }
  __syncthreads();
  // W = Tm X, row block w
  {
    T* Wout = wsW + cidx * CH * K;
#pragma unroll
    for (int n = 0; n < K / 16; ++n) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      mma_blk<true, true, CH>(acc, sTm, LC, 16 * w, sXt, LC, 16 * n);
#pragma unroll
      for (int i = 0; i < 4; ++i) Wout[(16 * w + acc_row(i)) * K + 16 * n + acc_col()] = from_f<T>(acc[i]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T, int K, int BV, bool BWD>
__global__ __launch_bounds__(NTHR) void fwd_state_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const float* __restrict__ beta,
    const float* __restrict__ h0, T* __restrict__ o, float* __restrict__ hT, const T* __restrict__ wsTm,
    const T* __restrict__ wsP, const T* __restrict__ wsW, const float* __restrict__ wsGc, T* __restrict__ wsH,
    T* __restrict__ wsR, int T_, int H, int V, int NT, float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT;
  constexpr int NCT = BV / 16;                  // column tiles of a 64 x BV block
  constexpr int NST = (K / 16) * NCT;           // tiles of the K x BV state slab
  constexpr int SPW = NST / NWAVE;              // state tiles per wave
  static_assert(NST % NWAVE == 0, "state slab must split evenly over the waves");
  __shared__ __attribute__((aligned(16))) T sW[CH * LK];
  __shared__ __attribute__((aligned(16))) T sQ[BWD ? 1 : CH * LK];
  __shared__ __attribute__((aligned(16))) T sKdt[K * LC];
  __shared__ __attribute__((aligned(16))) T sTm[CH * LC];
  __shared__ __attribute__((aligned(16))) T sP[BWD ? 1 : CH * LC];
  __shared__ __attribute__((aligned(16))) T sVt[BV * LC];
  __shared__ __attribute__((aligned(16))) T sSt[BV * LK];
  __shared__ __attribute__((aligned(16))) T sRt[BV * LC];
  __shared__ float sG[CH], sB[CH];

  const int vb = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int v0 = vb * BV;
  const int tid = threadIdx.x, w = wave_id();
  const int64_t sbase = (int64_t)bh * K * V;

  f32x4 S[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
    const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 16 * mi + acc_row(i), vc = 16 * ni + acc_col();
      S[s][i] = h0 ? h0[sbase + (int64_t)d * V + v0 + vc] : 0.f;
    }
  }

  for (int c = 0; c < NT; ++c) {
    const int t0 = c * CH;
    const int nvalid = min(CH, T_ - t0);
    const int64_t row0 = ((int64_t)b * T_ + t0) * H + h;
    const int64_t cidx = (int64_t)bh * NT + c;
    g2s_rows(sW, LK, wsW + cidx * CH * K, (int64_t)K, CH, K, CH);
    g2s_rows(sTm, LC, wsTm + cidx * CH * CH, (int64_t)CH, CH, CH, CH);
    if constexpr (!BWD) {
      g2s_rows(sQ, LK, q + row0 * K, (int64_t)H * K, CH, K, nvalid);
      g2s_rows(sP, LC, wsP + cidx * CH * CH, (int64_t)CH, CH, CH, CH);
    }
    if (tid < CH) {
      sG[tid] = wsGc[cidx * CH + tid];
      sB[tid] = tid < nvalid ? beta[row0 + (int64_t)tid * H] : 0.f;
    }
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * mi + acc_row(i), vc = 16 * ni + acc_col();
        const T val = from_f<T>(S[s][i]);
        sSt[vc * LK + d] = val;
        if constexpr (BWD) wsH[cidx * K * V + (int64_t)d * V + v0 + vc] = val;
      }
    }
    __syncthreads();
    const float GC = sG[CH - 1];
    for (int idx = tid; idx < CH * K; idx += NTHR) {
      const int j = idx / K, d = idx - j * K;
      const float kv = j < nvalid ? to_f(k[(row0 + (int64_t)j * H) * K + d]) : 0.f;
      sKdt[d * LC + j] = from_f<T>(__expf(GC - sG[j]) * kv);
    }
    for (int idx = tid; idx < CH * BV; idx += NTHR) {
      const int j = idx / BV, n = idx - j * BV;
      const float vv = j < nvalid ? to_f(v[(row0 + (int64_t)j * H) * V + v0 + n]) : 0.f;
      sVt[n * LC + j] = from_f<T>(sB[j] * vv);
    }
    __syncthreads();

    f32x4 QS[BWD ? 1 : NCT];
#pragma unroll
    for (int n = 0; n < NCT; ++n) {
      f32x4 u = {0.f, 0.f, 0.f, 0.f}, ws = {0.f, 0.f, 0.f, 0.f};
      mma_blk<true, true, CH>(u, sTm, LC, 16 * w, sVt, LC, 16 * n);
      mma_blk<true, true, K>(ws, sW, LK, 16 * w, sSt, LK, 16 * n);
      if constexpr (!BWD) {
        QS[n] = f32x4{0.f, 0.f, 0.f, 0.f};
        mma_blk<true, true, K>(QS[n], sQ, LK, 16 * w, sSt, LK, 16 * n);
      }
      const f32x4 R = u - ws;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * w + acc_row(i), vc = 16 * n + acc_col();
        const T val = from_f<T>(R[i]);
        sRt[vc * LC + r] = val;
        if constexpr (BWD) wsR[(cidx * CH + r) * V + v0 + vc] = val;
      }
    }
    __syncthreads();
    if constexpr (!BWD) {
#pragma unroll
      for (int n = 0; n < NCT; ++n) {
        f32x4 pr = {0.f, 0.f, 0.f, 0.f};
        mma_blk<true, true, CH>(pr, sP, LC, 16 * w, sRt, LC, 16 * n);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * w + acc_row(i), vc = 16 * n + acc_col();
          if (r < nvalid)
            o[(row0 + (int64_t)r * H) * V + v0 + vc] = from_f<T>(scale * __expf(sG[r]) * QS[n][i] + pr[i]);
        }
      }
    }
    const float gC = __expf(GC);
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
      S[s] *= gC;
      mma_blk<true, true, CH>(S[s], sKdt, LC, 16 * mi, sRt, LC, 16 * ni);
    }
    __syncthreads();
  }
  if (hT) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int ti = w + NWAVE * s, mi = ti / NCT, ni = ti - mi * NCT;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * mi + acc_row(i), vc = 16 * ni + acc_col();
        hT[sbase + (int64_t)d * V + v0 + vc] = S[s][i];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T> constexpr int state_bv() { return 32; }

template <typename T, int K>
static hipError_t fwd_intra_k(const ChunkArgs& a) {
  dim3 grid(a.NT, a.B * a.H);
  fwd_intra_kernel<T, K><<<grid, NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), a.g, a.beta, static_cast<T*>(a.ws.Tm),
      static_cast<T*>(a.ws.P), static_cast<T*>(a.ws.W), a.ws.Gc, a.T, a.H, a.NT, a.scale);
  return hipGetLastError();
}

template <typename T, int K, bool BWD>
static hipError_t fwd_state_k(const ChunkArgs& a) {
  constexpr int BV = state_bv<T>();
  dim3 grid(a.V / BV, a.B * a.H);
  fwd_state_kernel<T, K, BV, BWD><<<grid, NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.v), a.beta, a.h0,
      static_cast<T*>(a.o), BWD ? nullptr : a.hT, static_cast<const T*>(a.ws.Tm), static_cast<const T*>(a.ws.P),
      static_cast<const T*>(a.ws.W), a.ws.Gc, static_cast<T*>(a.ws.hs), static_cast<T*>(a.ws.Rs), a.T, a.H, a.V,
      a.NT, a.scale);
  return hipGetLastError();
}

hipError_t launch_fwd_intra(const ChunkArgs& a) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return fwd_intra_k<bf16, 64>(a);
    if (a.K == 128) return fwd_intra_k<bf16, 128>(a);
  } else {
    if (a.K == 64) return fwd_intra_k<float, 64>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fwd_state(const ChunkArgs& a, bool backward) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return backward ? fwd_state_k<bf16, 64, true>(a) : fwd_state_k<bf16, 64, false>(a);
    if (a.K == 128) return backward ? fwd_state_k<bf16, 128, true>(a) : fwd_state_k<bf16, 128, false>(a);
  } else {
    if (a.K == 64) return backward ? fwd_state_k<float, 64, true>(a) : fwd_state_k<float, 64, false>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace gdn
