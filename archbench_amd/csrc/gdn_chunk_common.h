// Per-chunk building blocks shared by the forward and backward chunk kernels.
//
// For one 64-token chunk of one head (local i, j; G = chunk-local cumsum of g, gamma = exp(G)):
//     A_ij = beta_i (k_i . k_j) exp(G_i - G_j)   (i > j)          Tm = (I + A)^-1  (unit lower triangular)
//     P_ij = s (q_i . k_j) exp(G_i - G_j)        (i >= j)
// (archbench/layers/nsgdn.py:240-249 with beta folded into the rows, as in the fla GDN chunk kernels it calls at
// nsgdn.py:357-362.)  The WY factors W = Tm diag(beta gamma) K and U = Tm diag(beta) V are never formed: with
// TmB = Tm diag(beta) the state sweeps use
//     R = U - W S = TmB (V - diag(gamma) K S)          and          W^T X = K^T diag(gamma) (TmB^T X),
// so K and V enter the MFMA products unscaled and no 64 x K factor is built per chunk.
#pragma once

#include "gdn_common.h"

namespace gdn {

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

// (I + A)^-1 for a strictly lower 64x64 A (fp32, LDS, stride LD) into the lower blocks of Ti (stride LD), in two
// stages so callers can overlap other work with the first:
//   invert_diag:   wave 0 only (others return at once) -- the four 16x16 diagonal blocks D_b by right-looking
//                  forward substitution, lane (b, c) solving column c of block b;
//   invert_merge:  all threads, after a barrier -- T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj by distance i - j on
//                  fp32 MFMA.  Ends with a barrier.
// Blocks above the diagonal of Ti are left untouched (callers treat them as zero).
template <int LD>
__device__ __forceinline__ void invert_diag(const float* A, float* Ti) {
  if (wave_id() != 0) return;
  const int l = lane_id();
  const int blk = l >> 4, cc = l & 15;
  const float* Ab = A + 16 * blk * LD + 16 * blk;
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
#pragma unroll
    for (int i = j + 1; i < 16; ++i) x[i] -= Ab[i * LD + j] * x[j];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) Ti[(16 * blk + i) * LD + 16 * blk + cc] = x[i];
}

template <int LD>
__device__ __forceinline__ void invert_merge(const float* A, float* Ti) {
  const int w = wave_id();
  auto blkp = [](const float* base, int i, int j) { return base + 16 * i * LD + 16 * j; };
  auto blkw = [](float* base, int i, int j) { return base + 16 * i * LD + 16 * j; };
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

template <int LD>
__device__ __forceinline__ void invert_unit_lower64(const float* A, float* Ti) {
  invert_diag<LD>(A, Ti);
  __syncthreads();
  invert_merge<LD>(A, Ti);
}

// A ROWS x COLS tile of T held in registers as 16-byte vectors (ROWS*COLS*sizeof(T)/16 split over NTHR threads),
// used to prefetch the next chunk while the current one is computed.  Loads are unconditional: rows past the
// end of the sequence read row 0 instead (always in bounds) and are zeroed only when the tile is stored, so no
// wait for the data is forced at load time.
template <typename T, int ROWS, int COLS>
struct RegTile {
  static constexpr int E = 16 / sizeof(T);
  static constexpr int VPR = COLS / E;
  static constexpr int N = ROWS * VPR / NTHR;
  static_assert(N * NTHR == ROWS * VPR && N >= 1 && N <= 32, "tile must split evenly over the workgroup");
  uint4 r[N];
  uint32_t ok;
  __device__ __forceinline__ void load(const T* g, int64_t gld, int valid) {
    ok = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = threadIdx.x + i * NTHR, row = idx / VPR, c = (idx - row * VPR) * E;
      const bool in = row < valid;
      ok |= (in ? 1u : 0u) << i;
      r[i] = *reinterpret_cast<const uint4*>(g + (in ? row : 0) * gld + c);
    }
  }
  __device__ __forceinline__ void store(T* s, int sld) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = threadIdx.x + i * NTHR, row = idx / VPR, c = (idx - row * VPR) * E;
      *reinterpret_cast<uint4*>(s + row * sld + c) = ((ok >> i) & 1u) ? r[i] : make_uint4(0, 0, 0, 0);
    }
  }
};

// Per-token scalars (g, beta) of a chunk for the first wave: same unconditional-load scheme.
struct RegTok {
  float g, b;
  bool ok;
  __device__ __forceinline__ void load(const float* pg, const float* pb, int64_t row0, int64_t stride, int valid) {
    const int l = threadIdx.x & 63;
    ok = l < valid;
    const int64_t off = row0 + (ok ? l : 0) * stride;
    g = pg[off];
    b = pb[off];
  }
};

// Copy a rows x cols tile from LDS (stride sld) to global (row stride gld), 16-byte vectors, rows < valid only.
template <typename T>
__device__ __forceinline__ void s2g_rows(T* g, int64_t gld, const T* s, int sld, int rows, int cols, int valid) {
  constexpr int E = 16 / sizeof(T);
  const int vpr = cols / E;
  for (int idx = threadIdx.x; idx < rows * vpr; idx += NTHR) {
    const int r = idx / vpr, c = (idx - r * vpr) * E;
    if (r < valid) *reinterpret_cast<uint4*>(g + r * gld + c) = *reinterpret_cast<const uint4*>(s + r * sld + c);
  }
}

// Chunk factors in LDS, phase 1 (all threads): K K^T and Q K^T on MFMA (row block = wave), then
//   A_ij = beta_i (K K^T)_ij exp(G_i - G_j) (i > j) -> sScr[0 : CH*LF]  (fp32, strict lower)
//   P_ij = s (Q K^T)_ij exp(G_i - G_j) (i >= j)     -> sP  (PMODE 1: [i][j];  PMODE 2: P^T, [j][i])
// then a barrier and the diagonal-block solve of the inverse on wave 0.  Waves 1-3 return immediately, so
// the caller can overlap independent work before calling chunk_factors_finish (which starts with a barrier).
// Inputs: sK (and sQ if PMODE != 0) rows of the chunk, zero past the sequence end; sG (cumulative log-decay);
// sB (beta, zero past the end).  sScr holds 2 * CH * LF floats.
template <typename T, int K, int PMODE>
__device__ __forceinline__ void chunk_factors_start(const T* sK, const T* sQ, const float* sG, const float* sB,
                                                    float scale, float* sScr, T* sP) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LF = CH + 4;
  const int w = wave_id();
  float* sA = sScr;
  // masks are selects on values computed unconditionally (exp of min(G_i - G_j, 0) cannot overflow), so the
  // epilogue has no branches around its LDS reads
  float Gr[4], Br[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    Gr[i] = sG[16 * w + acc_row(i)];
    Br[i] = sB[16 * w + acc_row(i)];
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
    mma_blk<true, true, K>(kk, sK, LK, 16 * w, sK, LK, 16 * n);
    if constexpr (PMODE != 0) mma_blk<true, true, K>(qk, sQ, LK, 16 * w, sK, LK, 16 * n);
    const int cc = 16 * n + acc_col();
    const float Gc = sG[cc];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i);
      const float e = __expf(fminf(Gr[i] - Gc, 0.f));
      const float a = Br[i] * kk[i] * e;
      const float p = scale * qk[i] * e;
      sA[r * LF + cc] = r > cc ? a : 0.f;
      if constexpr (PMODE == 1) sP[r * LC + cc] = from_f<T>(r >= cc ? p : 0.f);
      if constexpr (PMODE == 2) sP[cc * LC + r] = from_f<T>(r >= cc ? p : 0.f);
    }
  }
  __syncthreads();
  invert_diag<LF>(sA, sScr + CH * LF);
}

// Phase 2 (all threads): off-diagonal blocks of the inverse, then
//   TmB = Tm diag(beta)  -> sTmB  (TMODE 1: [i][j];  TMODE 2: TmB^T, [j][i])
//   Tm (unscaled)        -> gTm (global, 64 x 64 row-major) if non-null.
// Ends with a barrier; sScr is free again afterwards.
template <typename T, int TMODE>
__device__ __forceinline__ void chunk_factors_finish(const float* sB, float* sScr, T* sTmB, T* gTm) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LC = CH + PT, LF = CH + 4;
  __syncthreads();
  invert_merge<LF>(sScr, sScr + CH * LF);
  const float* sT = sScr + CH * LF;
  for (int idx = threadIdx.x; idx < CH * CH; idx += NTHR) {
    const int r = idx >> 6, cc = idx & 63;
    const float tv = sT[r * LF + cc];  // blocks above the diagonal are never written: masked below
    const float t = (r >> 4) >= (cc >> 4) ? tv : 0.f;
    if constexpr (TMODE == 1) sTmB[r * LC + cc] = from_f<T>(t * sB[cc]);
    else sTmB[cc * LC + r] = from_f<T>(t * sB[cc]);
    if (gTm) gTm[idx] = from_f<T>(t);
  }
  __syncthreads();
}

}  // namespace gdn
