// Chunkwise gated delta rule, forward sweep (fused): one workgroup per (64-wide V block, b*h), sequential over
// the 64-token chunks of the sequence.
//
// Per chunk (archbench/layers/nsgdn.py:240-249 algebra; fla GDN call order cumsum -> WY -> state -> output,
// nsgdn.py:357-362), everything stays on-chip:
//   chunk factors  K K^T, Q K^T on MFMA, A and P, the 64x64 inverse, TmB = Tm diag(beta) (rebuilt per V block,
//                  never written to HBM);
//   state part     one 16-column slab of S per wave, fp32 in MFMA accumulators for the whole sweep:
//                    R = TmB (V - diag(gamma) K S),  O = s gamma (Q S) + P R,
//                    S <- gamma_C S + K^T (exp(G_C - G) R)
//                  S and R reach the next product as B operands straight from the accumulators (permuted-k
//                  fragments), so waves never exchange state; only the chunk inputs are shared through LDS.
//
// bf16 (the training path) runs eight waves in two roles, two waves per SIMD, over two LDS buffer sets:
//   waves 0-3  state part of chunk c (buffer set n), one 16-column slab of S each; they also stage V (and Q)
//   waves 4-7  chunk factors of chunk c+1 (buffer set n^1); they also stage K, g, beta and scan g
// The two roles share the workgroup barriers (three per chunk) but never each other's data within a chunk, so
// each SIMD interleaves a latency-bound state wave with a latency-bound factor wave:
//   P1  state: stage V/Q of c+1, K S, Q S, Y of c       | factors: stage K/g/beta of c+1, g scan
//   P2  state: R, P R, O of c (staged)                   | factors: K K^T, Q K^T, diagonal inverse blocks of c+1
//   P3  state: O store, S update of c                    | factors: off-diagonal inverse blocks of c+1
// fp32 inputs (parity runs) do not fit two buffer sets in LDS; four waves run both roles for one chunk at a time.
// MODE 0 writes O; MODE 1 (recompute for the backward) writes instead, per chunk, the entering state and R (in
// the fragment layout, straight from the accumulators) and, from the first V block, Tm and G for the gradient
// kernels; MODE 2 (training forward) writes both, so that the backward needs no recompute.
#include "gdn_chunk_common.h"
#include "gdn_launch.h"

namespace gdn {

template <typename T, int K, int BV, int MODE, bool WS>
__global__ __launch_bounds__(WS ? 2 * NTHR : NTHR) void fwd_sweep_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ beta, const float* __restrict__ h0, T* __restrict__ o, float* __restrict__ hT,
    T* __restrict__ wsH, T* __restrict__ wsR, T* __restrict__ wsTm, float* __restrict__ wsGc, int T_, int H,
    int V, int NT, float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LV = BV + PT;
  constexpr int NKT = K / 16;           // row tiles of the state slab
  constexpr int NCW = BV / 16 / NWAVE;  // column tiles per state wave
  static_assert(NCW == 1, "each state wave owns one 16-column slab of the state");
  constexpr int NB = WS ? 2 : 1;       // LDS buffer sets
  constexpr bool OUT = MODE != 1;      // O is computed (needs Q and P)
  constexpr bool SAVE = MODE != 0;     // per-chunk states, R, Tm, G are written
  constexpr int PMODE = OUT ? 1 : 0;
  constexpr int STG = OUT ? CH * LV : 8;  // O staging
  __shared__ __attribute__((aligned(16))) T sK[NB][CH * LK];
  __shared__ __attribute__((aligned(16))) T sQ[NB][OUT ? CH * LK : 8];
  __shared__ __attribute__((aligned(16))) T sV[NB][CH * LV];
  __shared__ __attribute__((aligned(16))) T sP[NB][OUT ? CH * LC : 8];
  __shared__ __attribute__((aligned(16))) T sTmB[NB][CH * LC];
  __shared__ __attribute__((aligned(16))) float sA[CH * (CH + 4)];
  __shared__ __attribute__((aligned(16))) float sD[4 * DBLK];
  __shared__ __attribute__((aligned(16))) T stage[STG];
  __shared__ float sG[NB][CH], sB[NB][CH], sGam[NB][CH];

  int vb, bh;
  sweep_block(V / BV, gridDim.x * BV / V, vb, bh);
  const int b = bh / H, h = bh - b * H;
  const int v0 = vb * BV;
  const int w = wave_id(), l = lane_id();
  const int wr = w & (NWAVE - 1);            // wave index inside its role
  const int tid = threadIdx.x & (NTHR - 1);  // thread index inside its role
  const int64_t sbase = (int64_t)bh * K * V;
  auto row0_of = [&](int c) { return ((int64_t)b * T_ + (int64_t)c * CH) * H + h; };
  auto nvalid_of = [&](int c) { return min(CH, T_ - c * CH); };
  auto gtm_of = [&](int c) -> T* { return (SAVE && vb == 0) ? wsTm + ((int64_t)bh * NT + c) * CH * CH : nullptr; };
  const int ncb = V / 16, cb = vb * (BV / 16) + wr;  // fragment-layout column block of a state wave

  // ---- factor role: K, g, beta of a chunk, and its factors --------------------------------------------------
  RegTile<T, CH, K> rk;
  RegTok rt;
  auto prefetch_f = [&](int c) {
    rk.load(k + row0_of(c) * K, (int64_t)H * K, nvalid_of(c), tid);
    if (wr == 0) rt.load(g, beta, row0_of(c), H, nvalid_of(c));
  };
  auto store_f = [&](int c, int n) {
    rk.store(sK[n], LK, tid);
    if (wr == 0) {
      const float G = wave_inclusive_scan(rt.ok ? rt.g : 0.f);
      sG[n][l] = G;
      sB[n][l] = rt.ok ? rt.b : 0.f;
      sGam[n][l] = __expf(G);
      if (SAVE && vb == 0) wsGc[((int64_t)bh * NT + c) * CH + l] = G;
    }
  };
  auto kq_diag = [&](int c, int n) {
    factors_kq<T, K, PMODE>(sK[n], sQ[n], sG[n], sB[n], scale, sA, sP[n], wr);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the diagonal block reads this wave's rows of A
    return factors_diag<T>(sA, sD, sTmB[n], gtm_of(c), sB[n], wr);
  };

  // ---- state role: V (and Q) of a chunk, and the state part -------------------------------------------------
  RegTile<T, CH, K> rq;
  RegTile<T, CH, BV> rv;
  auto prefetch_s = [&](int c) {
    if constexpr (OUT) rq.load(q + row0_of(c) * K, (int64_t)H * K, nvalid_of(c), tid);
    rv.load(v + row0_of(c) * V + v0, (int64_t)H * V, nvalid_of(c), tid);
  };
  auto store_s = [&](int n) {
    if constexpr (OUT) rq.store(sQ[n], LK, tid);
    rv.store(sV[n], LV, tid);
  };
  const int c0 = 16 * wr;  // the state wave's column slab inside the V block
  f32x4 S[NKT];
  f32x4 Y[4], QS[4];
  typename Frag<T>::type Rd[2];
  auto load_h0 = [&]() {
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        S[t][i] = h0 ? h0[sbase + (int64_t)(16 * t + acc_row(i)) * V + v0 + c0 + acc_col()] : 0.f;
  };
  // K S, Q S and Y = V - diag(gamma) K S of the chunk in buffer set n (the entering state saved if SAVE)
  auto state_C = [&](int c, int n) {
    typename Frag<T>::type Sb[K / 32];
#pragma unroll
    for (int s = 0; s < K / 32; ++s) Sb[s] = frag_acc2<T>(S[2 * s], S[2 * s + 1]);
    if constexpr (SAVE) {
#pragma unroll
      for (int s = 0; s < K / 32; ++s) store_fragblk<T>(wsH + ((int64_t)bh * NT + c) * K * V, s, cb, ncb, Sb[s]);
    }
#pragma unroll
    for (int rt_ = 0; rt_ < 4; ++rt_) {
      f32x4 ks = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < K / 32; ++s) mma(ks, frag_kc_perm(sK[n], LK, 16 * rt_, 32 * s), Sb[s]);
      if constexpr (OUT) {
        QS[rt_] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < K / 32; ++s) mma(QS[rt_], frag_kc_perm(sQ[n], LK, 16 * rt_, 32 * s), Sb[s]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rt_ + acc_row(i);
        Y[rt_][i] = to_f(sV[n][r * LV + c0 + acc_col()]) - sGam[n][r] * ks[i];
      }
    }
  };
  // R = TmB Y (saved if SAVE); O = s gamma QS + P R staged
  auto state_D = [&](int c, int n) {
    typename Frag<T>::type Yb[2], Rb[2];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) Yb[jb] = frag_acc2<T>(Y[2 * jb], Y[2 * jb + 1]);
    f32x4 R[4];
#pragma unroll
    for (int rt_ = 0; rt_ < 4; ++rt_) {
      R[rt_] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) mma(R[rt_], frag_kc_perm(sTmB[n], LC, 16 * rt_, 32 * jb), Yb[jb]);
    }
    const float GC = sG[n][CH - 1];
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      f32x4 d0, d1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d0[i] = R[2 * jb][i] * __expf(GC - sG[n][32 * jb + acc_row(i)]);
        d1[i] = R[2 * jb + 1][i] * __expf(GC - sG[n][32 * jb + 16 + acc_row(i)]);
      }
      Rd[jb] = frag_acc2<T>(d0, d1);
      Rb[jb] = frag_acc2<T>(R[2 * jb], R[2 * jb + 1]);
      if constexpr (SAVE) store_fragblk<T>(wsR + ((int64_t)bh * NT + c) * CH * V, jb, cb, ncb, Rb[jb]);
    }
    if constexpr (OUT) {
#pragma unroll
      for (int rt_ = 0; rt_ < 4; ++rt_) {
        f32x4 pr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) mma(pr, frag_kc_perm(sP[n], LC, 16 * rt_, 32 * jb), Rb[jb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * rt_ + acc_row(i);
          stage[r * LV + c0 + acc_col()] = from_f<T>(scale * sGam[n][r] * QS[rt_][i] + pr[i]);
        }
      }
    }
  };
  // staged O -> global; S <- gamma_C S + K^T Rd
  auto state_E = [&](int c, int n) {
    if constexpr (OUT) s2g_rows(o + row0_of(c) * V + v0, (int64_t)H * V, stage, LV, CH, BV, nvalid_of(c));
    const float gC = __expf(sG[n][CH - 1]);
#pragma unroll
    for (int t = 0; t < NKT; ++t) {
      S[t] *= gC;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) mma(S[t], frag_oct_perm(sK[n], LK, 16 * t, 32 * jb), Rd[jb]);
    }
  };
  auto store_hT = [&]() {
    if (hT) {
#pragma unroll
      for (int t = 0; t < NKT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          hT[sbase + (int64_t)(16 * t + acc_row(i)) * V + v0 + c0 + acc_col()] = S[t][i];
    }
  };

  if constexpr (WS) {
    // Both roles execute the same sequence of barriers: two in the prologue, then three per chunk.
    if (w >= NWAVE) {
      prefetch_f(0);
      store_f(0, 0);
      __syncthreads();  // chunk 0 inputs in buffer set 0
      prefetch_f(min(1, NT - 1));
      const f32x4 D0 = kq_diag(0, 0);
      __syncthreads();
      factors_merge<T>(D0, sA, sD, sTmB[0], gtm_of(0), sB[0], wr);
      for (int c = 0; c < NT; ++c) {
        const int nn = (c & 1) ^ 1;
        const bool next = c + 1 < NT;
        __syncthreads();  // P1: factors of c complete; buffer set nn free
        if (next) store_f(c + 1, nn);
        prefetch_f(min(c + 2, NT - 1));
        __syncthreads();  // P2: inputs of c+1 in buffer set nn
        f32x4 D = zero4();
        if (next) D = kq_diag(c + 1, nn);
        __syncthreads();  // P3: diagonal blocks of c+1 in sD
        if (next) factors_merge<T>(D, sA, sD, sTmB[nn], gtm_of(c + 1), sB[nn], wr);
      }
    } else {
      load_h0();
      prefetch_s(0);
      store_s(0);
      __syncthreads();
      prefetch_s(min(1, NT - 1));
      __syncthreads();
      for (int c = 0; c < NT; ++c) {
        const int n = c & 1, nn = n ^ 1;
        __syncthreads();  // P1
        if (c + 1 < NT) store_s(nn);
        prefetch_s(min(c + 2, NT - 1));
        state_C(c, n);
        __syncthreads();  // P2
        state_D(c, n);
        __syncthreads();  // P3
        state_E(c, n);
      }
      store_hT();
    }
  } else {
    load_h0();
    prefetch_f(0);
    prefetch_s(0);
    for (int c = 0; c < NT; ++c) {
      store_f(c, 0);
      store_s(0);
      __syncthreads();
      if (c + 1 < NT) {
        prefetch_f(c + 1);
        prefetch_s(c + 1);
      }
      const f32x4 D = kq_diag(c, 0);
      state_C(c, 0);
      __syncthreads();
      factors_merge<T>(D, sA, sD, sTmB[0], gtm_of(c), sB[0], wr);
      __syncthreads();
      state_D(c, 0);
      __syncthreads();
      state_E(c, 0);
      __syncthreads();
    }
    store_hT();
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T, int K, int MODE>
static hipError_t fwd_sweep_k(const ChunkArgs& a) {
  constexpr int BV = 64;
  constexpr bool WS = sizeof(T) == 2;
  dim3 grid(a.V / BV * a.B * a.H);
  fwd_sweep_kernel<T, K, BV, MODE, WS><<<grid, WS ? 2 * NTHR : NTHR, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.v), a.g, a.beta, a.h0,
      static_cast<T*>(a.o), MODE == 1 ? nullptr : a.hT, static_cast<T*>(a.ws.hs), static_cast<T*>(a.ws.Rs),
      static_cast<T*>(a.ws.Tm), a.ws.Gc, a.T, a.H, a.V, a.NT, a.scale);
  return hipGetLastError();
}

template <typename T, int K>
static hipError_t fwd_sweep_mode(const ChunkArgs& a, FwdMode mode) {
  switch (mode) {
    case FWD_OUT: return fwd_sweep_k<T, K, 0>(a);
    case FWD_RECOMPUTE: return fwd_sweep_k<T, K, 1>(a);
    default: return fwd_sweep_k<T, K, 2>(a);
  }
}

hipError_t launch_fwd(const ChunkArgs& a, FwdMode mode) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return fwd_sweep_mode<bf16, 64>(a, mode);
    if (a.K == 128) return fwd_sweep_mode<bf16, 128>(a, mode);
  } else {
    if (a.K == 64) return fwd_sweep_mode<float, 64>(a, mode);
  }
  return hipErrorInvalidValue;
}

}  // namespace gdn
