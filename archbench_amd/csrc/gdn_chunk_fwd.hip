// Chunkwise gated delta rule, forward sweep (fused): one workgroup per (64-wide V block, b*h), sequential over
// the 64-token chunks of the sequence.
//
// Per chunk (archbench/layers/nsgdn.py:240-249 algebra; fla GDN call order cumsum -> WY -> state -> output,
// nsgdn.py:357-362), everything stays on-chip:
//   1. the chunk's k, q, v rows (prefetched into registers during the previous chunk) go to LDS; wave 0 scans g;
//   2. chunk factors: K K^T, Q K^T on MFMA, A and P, the 64x64 inverse, TmB = Tm diag(beta) (recomputed per
//      V block, never written to HBM); while wave 0 solves the diagonal blocks of the inverse, every wave
//      already forms K S and Q S for its columns;
//   3. state part, one 16-column slab of S per wave, fp32 in MFMA accumulators for the whole sweep:
//        R = TmB (V - diag(gamma) K S),  O = s gamma (Q S) + P R,  S <- gamma_C S + K^T (exp(G_C - G) R)
//      S and R reach the next product as B operands straight from the accumulators (permuted-k fragments), so
//      waves never exchange state; only the chunk inputs are shared through LDS.
// Backward-recompute mode writes, per chunk, the entering state (bf16 [K][V]), R (bf16 [64][V]) and, from the
// first V block, Tm and G for the gradient kernels, instead of O.
#include "gdn_chunk_common.h"
#include "gdn_launch.h"

namespace gdn {

template <typename T, int K, int BV, bool BWD>
__global__ __launch_bounds__(NTHR) void fwd_fused_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ beta, const float* __restrict__ h0, T* __restrict__ o, float* __restrict__ hT,
    T* __restrict__ wsH, T* __restrict__ wsR, T* __restrict__ wsTm, float* __restrict__ wsGc, int T_, int H,
    int V, int NT, float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LV = BV + PT, LF = CH + 4;
  constexpr int NKT = K / 16;           // row tiles of the state slab
  constexpr int NCW = BV / 16 / NWAVE;  // column tiles per wave
  static_assert(NCW == 1, "each wave owns one 16-column slab of the state");
  constexpr int SCR_F = 2 * CH * LF;  // fp32 scratch (A / inverse; then output staging)
  static_assert(SCR_F * 4 >= (BWD ? K : CH) * LV * (int)sizeof(T), "staging must fit in the scratch region");
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];
  __shared__ __attribute__((aligned(16))) T sQ[BWD ? 8 : CH * LK];
  __shared__ __attribute__((aligned(16))) T sV[CH * LV];
  __shared__ __attribute__((aligned(16))) T sP[BWD ? 8 : CH * LC];
  __shared__ __attribute__((aligned(16))) T sTmB[CH * LC];
  __shared__ __attribute__((aligned(16))) float sScr[SCR_F];
  __shared__ float sG[CH], sB[CH], sGam[CH];

  const int vb = blockIdx.x, bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const int v0 = vb * BV;
  const int w = wave_id(), l = lane_id();
  const int c0 = 16 * w;  // this wave's column slab inside the V block
  const int64_t sbase = (int64_t)bh * K * V;
  T* stage = reinterpret_cast<T*>(sScr);

  f32x4 S[NKT];
#pragma unroll
  for (int t = 0; t < NKT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[t][i] = h0 ? h0[sbase + (int64_t)(16 * t + acc_row(i)) * V + v0 + c0 + acc_col()] : 0.f;

  RegTile<T, CH, K> rk, rq;
  RegTile<T, CH, BV> rv;
  RegTok rt;
  auto prefetch = [&](int c) {
    const int t0 = c * CH, nvalid = min(CH, T_ - t0);
    const int64_t row0 = ((int64_t)b * T_ + t0) * H + h;
    rk.load(k + row0 * K, (int64_t)H * K, nvalid);
    if constexpr (!BWD) rq.load(q + row0 * K, (int64_t)H * K, nvalid);
    rv.load(v + row0 * V + v0, (int64_t)H * V, nvalid);
    if (w == 0) rt.load(g, beta, row0, H, nvalid);
  };
  prefetch(0);

  for (int c = 0; c < NT; ++c) {
    const int t0 = c * CH, nvalid = min(CH, T_ - t0);
    const int64_t row0 = ((int64_t)b * T_ + t0) * H + h;
    const int64_t cidx = (int64_t)bh * NT + c;
    rk.store(sK, LK);
    if constexpr (!BWD) rq.store(sQ, LK);
    rv.store(sV, LV);
    if (w == 0) {
      const float G = wave_inclusive_scan(rt.ok ? rt.g : 0.f);
      sG[l] = G;
      sB[l] = rt.ok ? rt.b : 0.f;
      sGam[l] = __expf(G);
      if (BWD && vb == 0) wsGc[cidx * CH + l] = G;
    }
    __syncthreads();
    if (c + 1 < NT) prefetch(c + 1);

    T* gTm = (BWD && vb == 0) ? wsTm + cidx * CH * CH : nullptr;
    const f32x4 Dw = chunk_factors_start<T, K, BWD ? 0 : 1>(sK, sQ, sG, sB, scale, sScr, sP, sTmB, gTm);
    // independent of the inverse (overlaps its latency):  K S and Q S for this wave's columns, Y = V - gamma K S
    typename Frag<T>::type Sb[K / 32];
#pragma unroll
    for (int s = 0; s < K / 32; ++s) Sb[s] = frag_acc2<T>(S[2 * s], S[2 * s + 1]);
    f32x4 Y[4], QS[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4 ks = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < K / 32; ++s) mma(ks, frag_kc_perm(sK, LK, 16 * rt, 32 * s), Sb[s]);
      if constexpr (!BWD) {
        QS[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < K / 32; ++s) mma(QS[rt], frag_kc_perm(sQ, LK, 16 * rt, 32 * s), Sb[s]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rt + acc_row(i);
        Y[rt][i] = to_f(sV[r * LV + c0 + acc_col()]) - sGam[r] * ks[i];
      }
    }
    chunk_factors_finish<T>(Dw, sB, sScr, sTmB, gTm);

    // ---- R = TmB Y, output, state update (this wave's 16 columns) ------------------------------------------
    typename Frag<T>::type Yb[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) Yb[jb] = frag_acc2<T>(Y[2 * jb], Y[2 * jb + 1]);
    f32x4 R[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      R[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) mma(R[rt], frag_kc_perm(sTmB, LC, 16 * rt, 32 * jb), Yb[jb]);
    }
    const float GC = sG[CH - 1];
    typename Frag<T>::type Rb[2], Rd[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      f32x4 d0, d1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d0[i] = R[2 * jb][i] * __expf(GC - sG[32 * jb + acc_row(i)]);
        d1[i] = R[2 * jb + 1][i] * __expf(GC - sG[32 * jb + 16 + acc_row(i)]);
      }
      Rd[jb] = frag_acc2<T>(d0, d1);
      if constexpr (!BWD) Rb[jb] = frag_acc2<T>(R[2 * jb], R[2 * jb + 1]);
    }
    if constexpr (BWD) {
      // entering state -> global h (bf16 [K][V] per chunk); R -> global (bf16 [64][V] per chunk)
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) stage[(16 * t + acc_row(i)) * LV + c0 + acc_col()] = from_f<T>(S[t][i]);
      __syncthreads();
      s2g_rows(wsH + cidx * K * V + v0, (int64_t)V, stage, LV, K, BV, K);
      __syncthreads();
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) stage[(16 * rt + acc_row(i)) * LV + c0 + acc_col()] = from_f<T>(R[rt][i]);
      __syncthreads();
      s2g_rows(wsR + cidx * CH * V + v0, (int64_t)V, stage, LV, CH, BV, CH);
    } else {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        f32x4 pr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) mma(pr, frag_kc_perm(sP, LC, 16 * rt, 32 * jb), Rb[jb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * rt + acc_row(i);
          stage[r * LV + c0 + acc_col()] = from_f<T>(scale * sGam[r] * QS[rt][i] + pr[i]);
        }
      }
      __syncthreads();
      s2g_rows(o + row0 * V + v0, (int64_t)H * V, stage, LV, CH, BV, nvalid);
    }
    // S <- gamma_C S + K^T (exp(G_C - G) R)
    const float gC = __expf(GC);
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
      S[t] *= gC;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) mma(S[t], frag_oct_perm(sK, LK, 16 * t, 32 * jb), Rd[jb]);
    }
    __syncthreads();
  }
  if (hT) {
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) hT[sbase + (int64_t)(16 * t + acc_row(i)) * V + v0 + c0 + acc_col()] = S[t][i];
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T, int K, bool BWD>
static hipError_t fwd_fused_k(const ChunkArgs& a) {
  constexpr int BV = 64;
  dim3 grid(a.V / BV, a.B * a.H);
  fwd_fused_kernel<T, K, BV, BWD><<<grid, NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.v), a.g, a.beta, a.h0,
      static_cast<T*>(a.o), BWD ? nullptr : a.hT, static_cast<T*>(a.ws.hs), static_cast<T*>(a.ws.Rs),
      static_cast<T*>(a.ws.Tm), a.ws.Gc, a.T, a.H, a.V, a.NT, a.scale);
  return hipGetLastError();
}

hipError_t launch_fwd(const ChunkArgs& a, bool backward) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return backward ? fwd_fused_k<bf16, 64, true>(a) : fwd_fused_k<bf16, 64, false>(a);
    if (a.K == 128) return backward ? fwd_fused_k<bf16, 128, true>(a) : fwd_fused_k<bf16, 128, false>(a);
  } else {
    if (a.K == 64) return backward ? fwd_fused_k<float, 64, true>(a) : fwd_fused_k<float, 64, false>(a);
  }
  return hipErrorInvalidValue;
}

}  // namespace gdn
