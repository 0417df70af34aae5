// Chunkwise gated delta rule, forward state sweep: one workgroup per (V block of 64 columns, or 32 when the grid
// fits the device, b*h), sequential over the 64-token chunks of the sequence, after the chunk factors (Tm, P, G)
// have been built for all chunks in parallel (gdn_chunk_factors.hip).
//
// Per chunk (archbench/layers/nsgdn.py:240-249 algebra; fla GDN call order cumsum -> WY -> state -> output,
// nsgdn.py:357-362), each wave holds one 16-column slab of S in fp32 MFMA accumulators for the whole sweep:
//     Y = diag(beta) (V - diag(gamma) K S)          R = Tm Y            (= U - W S)
//     O = s diag(gamma) Q S + P R                   S <- gamma_C S + K^T (exp(G_C - G) R)
// S, Y and R reach the next product as B operands straight from the accumulators (permuted-k fragments); the
// chunk inputs are shared through LDS, and so is half of each wave's state slab (below).  The next chunk's
// inputs are prefetched into registers one chunk ahead.
// MODE 0 writes O (and hT); MODE 1 (recompute for the backward) writes instead the state entering every chunk
// (every hstride-th) and R, in the fragment layout straight from the accumulators; MODE 2 (training forward)
// writes both.
// MODE 3 (the prefix pass of a segmented sweep) writes only the final state, and the grid carries K more columns
// per head: those "identity" blocks start from S = I with V = 0, so their final state is the segment's transition
// Phi = prod_c (gamma_C I - K^T diag(exp(G_C - G)) Tm diag(beta gamma) K), written to phi [BH][K][K].  The
// first segment of each sequence starts from h0 instead of zero, so its "local" state already carries h0 and its
// Phi is never needed; nor is the last segment's state (the main sweep writes hT) or its Phi (the local reverse
// pass starts that segment from dhT): those blocks return at once.
// SEPU (separate write keys u, nsgdn.py:240-249): the state update is S <- gamma_C S + U^T (exp(G_C - G) R) with
// U loaded beside K; K keeps the read K S; beta may be absent (row scale 1).
#include "gdn_chunk_common.h"
#include "gdn_launch.h"

namespace gdn {

// Two waves per 16-column slab of the V block (BV / 16 slabs: eight waves for BV = 64, four for BV = 32).  Waves
// w and w + NSL share the slab 16 (w % NSL); the chunk's token rows are split between them (half hf = w / NSL
// takes rows 32 hf .. 32 hf + 31, i.e. the permuted-k fragment hf of every token-indexed product), and so are
// the state's K rows (wave hf holds and updates rows K/2 hf .. K/2 hf + K/2 - 1 of the slab).  Each half computes
// K S, Q S, Y, R, P R and O for its token rows; the Y and Rd fragments of the other half come through LDS (16
// bytes per lane each), and so do the bf16 fragments of the other half's state rows, written after the update
// and read after the next chunk's first barrier (no barrier of their own).
template <int BV>
constexpr int fwd_threads() { return 128 * (BV / 16); }
constexpr bool FWD_NT_LOAD = true;             // chunk inputs (measured faster with the hint)
constexpr bool FWD_NT_STORE = true;            // O, and the stashed states and R: written once

template <typename T, int K, int BV, int MODE, bool SEPU>
__global__ __launch_bounds__(fwd_threads<BV>()) __attribute__((amdgpu_waves_per_eu(2))) void fwd_sweep_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ u, const T* __restrict__ v,
    const float* __restrict__ beta,
    const float* __restrict__ h0, const T* __restrict__ gTm, const T* __restrict__ gP,
    const float* __restrict__ gGc, T* __restrict__ o, float* __restrict__ hT, float* __restrict__ phi,
    T* __restrict__ wsH, T* __restrict__ wsR, int T_, int H, int V, int NT, float scale, int ns, int hstride) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LV = BV + PT;
  constexpr int NKT = K / 16;  // row tiles of the state slab
  constexpr int NKH = NKT / 2, NSB = K / 64;  // row tiles and 32-row fragments held by each wave of the pair
  constexpr int NSL = BV / 16, FW = 2 * NSL, FTH = 64 * FW;  // slabs, waves, threads
  static_assert(NSL == 2 || NSL == 4, "a wave pair per 16-column slab, two or four slabs");
  constexpr bool OUT = MODE == 0 || MODE == 2;   // O is computed (needs Q and P)
  constexpr bool SAVE = MODE == 1 || MODE == 2;  // per-chunk states and R are written
  using F = typename Frag<T>::type;
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];
  __shared__ __attribute__((aligned(16))) T sU_[SEPU ? CH * LK : 8];
  T* sU = SEPU ? sU_ : sK;  // write keys
  __shared__ __attribute__((aligned(16))) T sQ[OUT ? CH * LK : 8];
  __shared__ __attribute__((aligned(16))) T sV[CH * LV];
  __shared__ __attribute__((aligned(16))) T sTm[CH * LC];
  __shared__ __attribute__((aligned(16))) T sP[OUT ? CH * LC : 8];
  __shared__ __attribute__((aligned(16))) T stage[OUT ? CH * LV : 8];  // O, for the coalesced store
  __shared__ __attribute__((aligned(16))) F xY[FW][64], xR[FW][64], xRd[FW][64];  // exchange between halves
  // the other half's state fragments, in the reading wave's slot.  fp32 (K = 64: one fragment) uses the reader's Y
  // slot: the writer reads the reader's Y there (after the Y exchange barrier) before it writes the state after the
  // update, and the reader writes its next Y there only after it has read the state.
  constexpr bool S_ON_Y = sizeof(T) == 4;
  static_assert(!S_ON_Y || NSB == 1, "the state fragments fit one exchange slot");
  __shared__ __attribute__((aligned(16))) F xS_[S_ON_Y ? 1 : FW][NSB][64];
  auto xS = [&](int wr, int s) -> F& {
    if constexpr (S_ON_Y) return xY[wr][lane_id()];
    else return xS_[wr][s][lane_id()];
  };
  // per token: beta, exp(G), exp(G_C - G), s exp(G) (formed once per chunk by the first wave)
  __shared__ float sB[CH], sGam[CH], sDte[CH], sGs[CH];

  int vb, bh;
  const int NVB = (V + (MODE == 3 ? K : 0)) / BV;  // column blocks per head
  sweep_block(NVB, gridDim.x / NVB, vb, bh);
  const int b = bh / H, h = bh - b * H;
  // identity block (MODE 3): columns iv0 .. iv0 + BV - 1 of the transition; v reads nothing (no valid rows)
  const bool ident = MODE == 3 && vb * BV >= V;
  const int iv0 = vb * BV - V;
  const int v0 = ident ? 0 : vb * BV;
  const int seg = b % ns;  // segment of sequence b / ns (ns = 1: not segmented)
  if constexpr (MODE == 3) {
    if (seg == ns - 1 || (ident && seg == 0)) return;  // uniform over the workgroup, before any barrier
  }
  // hT: per swept sequence in MODE 3 (the segments' local states); otherwise, when segmented, only from the last
  // segment of each sequence, at the sequence's index.  h0: in MODE 3 the sequence's own, for its first segment
  // only; otherwise per swept sequence (the entering state of every segment).
  const bool put_hT = MODE == 3 || seg == ns - 1;
  const int64_t hT_base = (MODE == 3 ? (int64_t)bh : (int64_t)(b / ns) * H + h) * K * V;
  const bool use_h0 = h0 && (MODE != 3 || seg == 0);
  const int64_t h0_base = (MODE == 3 ? (int64_t)(b / ns) * H + h : (int64_t)bh) * K * V;
  const int w = wave_id(), l = lane_id();
  const int ws = w & (NSL - 1), hf = w / NSL;        // column slab, token half
  const int c0 = 16 * ws;                             // the slab inside the V block
  const int ncb = V / 16, cb = vb * (BV / 16) + ws;  // its fragment-layout column block
  const int tid = threadIdx.x;
  auto row0_of = [&](int c) { return ((int64_t)b * T_ + (int64_t)c * CH) * H + h; };
  auto nvalid_of = [&](int c) { return min(CH, T_ - c * CH); };

  RegTile<T, CH, K, FTH, FWD_NT_LOAD> rk, rq, ru;
  RegTile<T, CH, BV, FTH, FWD_NT_LOAD> rv;
  TriTile<T, FTH, FWD_NT_LOAD> rtm, rp;  // packed lower blocks
  float pG = 0.f, pB = 0.f;  // wave 0: G and beta of lane l's token
  // The next chunk's reads go out in two batches (k, q, v after the first barrier; Tm, P, G, beta after the
  // second exchange), so that no wave stalls on a full memory queue for the whole set at once.
  auto prefetch = [&](int c) {
    const int64_t row0 = row0_of(c);
    const int nv = nvalid_of(c);
    rk.load(k + row0 * K, (int64_t)H * K, nv, tid);
    if constexpr (SEPU) ru.load(u + row0 * K, (int64_t)H * K, nv, tid);
    if constexpr (OUT) rq.load(q + row0 * K, (int64_t)H * K, nv, tid);
    rv.load(v + row0 * V + v0, (int64_t)H * V, ident ? 0 : nv, tid);
  };
  auto prefetch2 = [&](int c) {
    const int64_t row0 = row0_of(c), cidx = (int64_t)bh * NT + c;
    const int nv = nvalid_of(c);
    rtm.load(gTm + cidx * CH_TRI_ELEMS, tid);
    if constexpr (OUT) rp.load(gP + cidx * CH_TRI_ELEMS, tid);
    if (w == 0) {
      pG = gGc[cidx * CH + l];
      pB = l < nv ? (beta ? beta[row0 + (int64_t)l * H] : 1.f) : 0.f;
    }
  };
  auto to_lds = [&]() {
    rk.store(sK, LK, tid);
    if constexpr (SEPU) ru.store(sU, LK, tid);
    if constexpr (OUT) rq.store(sQ, LK, tid);
    rv.store(sV, LV, tid);
    rtm.store(sTm, LC, tid);
    if constexpr (OUT) rp.store(sP, LC, tid);
    if (w == 0) {
      const float gam = __expf(pG), GCl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pG), CH - 1));
      sB[l] = pB;
      sGam[l] = gam;
      sDte[l] = __expf(GCl - pG);
      sGs[l] = scale * gam;
    }
  };

  f32x4 S[NKH];  // state rows 16 (NKH hf + t) .. + 15 of the slab
#pragma unroll
  for (int t = 0; t < NKH; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * (NKH * hf + t) + acc_row(i);
      S[t][i] = ident ? (row == iv0 + c0 + acc_col() ? 1.f : 0.f)
                      : (use_h0 ? h0[h0_base + (int64_t)row * V + v0 + c0 + acc_col()] : 0.f);
    }
  F Smine[NSB];  // bf16 fragments of the wave's state rows (32-row blocks NSB hf ..), also written to xS
  auto publish_state = [&]() {
#pragma unroll
    for (int s = 0; s < NSB; ++s) {
      Smine[s] = frag_acc2<T>(S[2 * s], S[2 * s + 1]);
      xS(w ^ NSL, s) = Smine[s];
    }
  };

  auto chunk = [&](int c) {
    const int64_t cidx = (int64_t)bh * NT + c;
    to_lds();
    __syncthreads();
    if (c + 1 < NT) prefetch(c + 1);

    // rows 32 hf .. 32 hf + 31: K S, Q S and Y = diag(beta) (V - diag(gamma) K S); the state's fragments are the
    // wave's own and, for the other half of the K rows, the partner's from xS (written before the last barrier).
    // Here and below a product over both halves pairs each fragment with the other operand's columns for its half
    // (offsets by hf), so no fragment is selected by the half.
    F Sother[NSB];
#pragma unroll
    for (int s = 0; s < NSB; ++s) Sother[s] = xS(w, s);
    const int kmine = (K / 2) * hf, kother = (K / 2) - kmine;  // first K column of each half
    // the state entering every hstride-th chunk goes to the stash (slot c / hstride of the sequence), each wave
    // its own rows; the branch is uniform and the stored values come from registers, not from loads in flight
    const bool keep = (c & (hstride - 1)) == 0;
    const int64_t hidx = (int64_t)bh * ((NT + hstride - 1) / hstride) + c / hstride;
    if constexpr (SAVE) {
      if (keep) {
#pragma unroll
        for (int s = 0; s < NSB; ++s)
          store_fragblk<T, FWD_NT_STORE>(wsH + hidx * K * V, K, NSB * hf + s, cb, ncb, Smine[s]);
      }
    }
    f32x4 Y[2], QS[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rt_ = 2 * hf + j;
      f32x4 ks = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NSB; ++s) mma(ks, frag_kc_perm(sK, LK, 16 * rt_, kmine + 32 * s), Smine[s]);
#pragma unroll
      for (int s = 0; s < NSB; ++s) mma(ks, frag_kc_perm(sK, LK, 16 * rt_, kother + 32 * s), Sother[s]);
      if constexpr (OUT) {
        QS[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NSB; ++s) mma(QS[j], frag_kc_perm(sQ, LK, 16 * rt_, kmine + 32 * s), Smine[s]);
#pragma unroll
        for (int s = 0; s < NSB; ++s) mma(QS[j], frag_kc_perm(sQ, LK, 16 * rt_, kother + 32 * s), Sother[s]);
      }
      float vv[4];
      acc_vals(sV, LV, 16 * rt_, c0, vv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rt_ + acc_row(i);
        Y[j][i] = sB[r] * (vv[i] - sGam[r] * ks[i]);
      }
    }
    const F Ymine = frag_acc2<T>(Y[0], Y[1]);
    xY[w][l] = Ymine;
    __syncthreads();
    const F Yother = xY[w ^ NSL][l];
    const int tmine = 32 * hf, tother = 32 - tmine;  // first token of each half

    // R = Tm Y for the half's rows (saved if SAVE); Rd = exp(G_C - G) R; O = s gamma QS + P R staged
    f32x4 R[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      R[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma(R[j], frag_kc_perm(sTm, LC, 16 * (2 * hf + j), tmine), Ymine);
      mma(R[j], frag_kc_perm(sTm, LC, 16 * (2 * hf + j), tother), Yother);
    }
    F Rdmine;
    {
      f32x4 d0, d1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d0[i] = R[0][i] * sDte[32 * hf + acc_row(i)];
        d1[i] = R[1][i] * sDte[32 * hf + 16 + acc_row(i)];
      }
      Rdmine = frag_acc2<T>(d0, d1);
      xRd[w][l] = Rdmine;
    }
    const F Rbmine = frag_acc2<T>(R[0], R[1]);
    if constexpr (OUT) xR[w][l] = Rbmine;
    if constexpr (SAVE) store_fragblk<T, FWD_NT_STORE>(wsR + cidx * CH * V, CH, hf, cb, ncb, Rbmine);
    __syncthreads();  // R and Rd fragments of both halves exchanged
    if (c + 1 < NT) prefetch2(c + 1);
    const F Rdother = xRd[w ^ NSL][l];
    if constexpr (OUT) {
      const F Rbother = xR[w ^ NSL][l];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int rt_ = 2 * hf + j;
        f32x4 pr = {0.f, 0.f, 0.f, 0.f};
        mma(pr, frag_kc_perm(sP, LC, 16 * rt_, tmine), Rbmine);
        mma(pr, frag_kc_perm(sP, LC, 16 * rt_, tother), Rbother);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * rt_ + acc_row(i);
          stage[r * LV + c0 + acc_col()] = from_f<T>(sGs[r] * QS[j][i] + pr[i]);
        }
      }
    }
    // S <- gamma_C S + U^T Rd for the wave's state rows (both halves of the chunk's tokens)
    const float gC = sGam[CH - 1];  // exp(G_C)
#pragma unroll
    for (int t = 0; t < NKH; ++t) {
      S[t] *= gC;
      mma(S[t], frag_oct_perm(sU, LK, 16 * (NKH * hf + t), tmine), Rdmine);
      mma(S[t], frag_oct_perm(sU, LK, 16 * (NKH * hf + t), tother), Rdother);
    }
    publish_state();  // the partner read the previous fragments before the exchange barriers above
    __syncthreads();  // O staged; every wave done with this chunk's inputs
    if constexpr (OUT)
      s2g_rows<T, CH, BV, FTH, FWD_NT_STORE>(o + row0_of(c) * V + v0, (int64_t)H * V, stage, LV, nvalid_of(c));
  };
  // the blocks of Tm and P above the diagonal stay zero (the packed loads write the others); ordered before any
  // read by the first chunk's first barrier
  tri_zero_upper<T, FTH>(sTm, LC, tid);
  if constexpr (OUT) tri_zero_upper<T, FTH>(sP, LC, tid);
  publish_state();  // read after the first chunk's first barrier
  prefetch(0);
  prefetch2(0);
  for (int c = 0; c < NT; ++c) chunk(c);
  if (ident) {
#pragma unroll
    for (int t = 0; t < NKH; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        phi[((int64_t)bh * K + 16 * (NKH * hf + t) + acc_row(i)) * K + iv0 + c0 + acc_col()] = S[t][i];
  } else if (hT && put_hT) {
#pragma unroll
    for (int t = 0; t < NKH; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        hT[hT_base + (int64_t)(16 * (NKH * hf + t) + acc_row(i)) * V + v0 + c0 + acc_col()] = S[t][i];
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T, int K, int MODE, bool SEPU, int BV>
static hipError_t fwd_sweep_bv(const ChunkArgs& a) {
  dim3 grid((a.V + (MODE == 3 ? K : 0)) / BV * a.B * a.H);
  fwd_sweep_kernel<T, K, BV, MODE, SEPU><<<grid, fwd_threads<BV>(), 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.u),
      static_cast<const T*>(a.v), a.beta, a.h0,
      static_cast<const T*>(a.ws.Tm), static_cast<const T*>(a.ws.P), a.ws.Gc, static_cast<T*>(a.o),
      MODE == 1 ? nullptr : a.hT, a.ws.phi, static_cast<T*>(a.ws.hs), static_cast<T*>(a.ws.Rs), a.T, a.H, a.V,
      a.NT, a.scale, a.ns, a.hstride);
  return hipGetLastError();
}

template <typename T, int K, int MODE, bool SEPU>
static hipError_t fwd_sweep_k(const ChunkArgs& a) {
  if constexpr (sizeof(T) == 2 && !SEPU) {
    if (narrow_sweep_blocks(a, (a.V + (MODE == 3 ? K : 0)) / 32)) return fwd_sweep_bv<T, K, MODE, SEPU, 32>(a);
  }
  return fwd_sweep_bv<T, K, MODE, SEPU, 64>(a);
}

template <typename T, int K>
static hipError_t fwd_sweep_mode(const ChunkArgs& a, FwdMode mode) {
  if constexpr (sizeof(T) == 2) {
    if (a.u) {  // separate write keys: the training pair only (stashing forward, and its prefix pass)
      if (mode == FWD_STASH) return fwd_sweep_k<T, K, 2, true>(a);
      if (mode == FWD_PREFIX) return fwd_sweep_k<T, K, 3, true>(a);
      return hipErrorInvalidValue;
    }
  }
  switch (mode) {
    case FWD_OUT: return fwd_sweep_k<T, K, 0, false>(a);
    case FWD_RECOMPUTE: return fwd_sweep_k<T, K, 1, false>(a);
    case FWD_PREFIX: return fwd_sweep_k<T, K, 3, false>(a);
    default: return fwd_sweep_k<T, K, 2, false>(a);
  }
}

hipError_t launch_fwd(const ChunkArgs& a, FwdMode mode) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return fwd_sweep_mode<bf16, 64>(a, mode);
    if (a.K == 128) return fwd_sweep_mode<bf16, 128>(a, mode);
  } else if (!a.u) {  // separate write keys: bf16 only
    if (a.K == 64) return fwd_sweep_mode<float, 64>(a, mode);
  }
  return hipErrorInvalidValue;
}

}  // namespace gdn
