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

#include <type_traits>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

// ---- 64x64 unit-lower-triangular inverse ------------------------------------------------------------------
// Blocked by 16.  Products are 16x16x16 on "slices": an A-slice holds, in lane l (g = l >> 4), A[l & 15][4g + j],
// a B-slice holds B[4g + j][l & 15] (j = 0..3), which is also the layout of a 16x16 fp32 accumulator.  The
// A-slice of X is therefore the accumulator of X^T, so a chain of products stays in registers as long as both
// X and X^T are carried.  fp32 inputs use four v_mfma_f32_16x16x4_f32; bf16 runs use the split
// x = hi + lo (hi = bf16(x), lo = bf16(x - hi)) and three v_mfma_f32_16x16x16_bf16 (hi hi, hi lo, lo hi),
// which keeps the inverse at about fp32 accuracy.
__device__ __forceinline__ void split_hi_lo(const f32x4& x, shortx4& hi, shortx4& lo) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16 h = static_cast<bf16>(x[j]);
    hi[j] = __builtin_bit_cast(short, h);
    lo[j] = __builtin_bit_cast(short, static_cast<bf16>(x[j] - static_cast<float>(h)));
  }
}
template <typename T>
__device__ __forceinline__ void mm16(f32x4& c, const f32x4& a, const f32x4& b) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  } else {
    shortx4 ah, al, bh, bl;
    split_hi_lo(a, ah, al);
    split_hi_lo(b, bh, bl);
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bl, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bh, c, 0, 0, 0);
  }
}
template <int LD>
__device__ __forceinline__ f32x4 ld_aslice(const float* p) {
  const int l = lane_id();
  return *reinterpret_cast<const f32x4*>(p + (l & 15) * LD + 4 * (l >> 4));
}
template <int LD>
__device__ __forceinline__ f32x4 ld_bslice(const float* p) {
  const int l = lane_id();
  f32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = p[(4 * (l >> 4) + j) * LD + (l & 15)];
  return r;
}
// s * I as a slice (the same lanes hold the diagonal in the A-slice and in the accumulator layout)
__device__ __forceinline__ f32x4 eye16(float s) {
  const int l = lane_id();
  f32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = (l & 15) == 4 * (l >> 4) + j ? s : 0.f;
  return r;
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Diagonal block D = (I + L)^-1 of a strictly lower 16x16 L (fp32 in LDS, stride LD), as an accumulator:
// L^16 = 0, so D = (I - L)(I + L^2)(I + L^4)(I + L^8).
template <typename T, int LD>
__device__ __forceinline__ f32x4 inv_diag16(const float* Lp) {
  const f32x4 La = ld_aslice<LD>(Lp), Lb = ld_bslice<LD>(Lp);  // L as A-slice; L as B-slice (= L^T A-slice)
  const f32x4 I = eye16(1.f);
  f32x4 L2 = zero4(), L2t = zero4(), L4 = zero4(), L4t = zero4(), L8 = zero4();
  mm16<T>(L2, La, Lb);    // L L
  mm16<T>(L2t, Lb, La);   // L^T L^T
  mm16<T>(L4, L2t, L2);   // L^2 L^2
  mm16<T>(L4t, L2, L2t);  // (L^2)^T (L^2)^T
  mm16<T>(L8, L4t, L4);   // L^4 L^4
  const f32x4 ImL = I - La;  // (I - L) A-slice  =  (I - L)^T B-slice
  f32x4 Z1t = zero4(), Z2t = zero4(), D = zero4();
  mm16<T>(Z1t, I + L2, ImL);   // Z1^T = (I + L^2)^T (I - L)^T
  mm16<T>(Z2t, I + L4, Z1t);   // Z2^T = (I + L^4)^T Z1^T
  mm16<T>(D, Z2t, I + L8);     // D = Z2 (I + L^8)
  return D;
}

// Writes block (bi, bj) of Tm (accumulator x) into LDS (row-major, stride LC).
template <typename T, int LC>
__device__ __forceinline__ void put_tm_block(T* sTm, int bi, int bj, const f32x4& x) {
  const int l = lane_id();
  const int col = 16 * bj + (l & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i) sTm[(16 * bi + 4 * (l >> 4) + i) * LC + col] = from_f<T>(x[i]);
}

// Compact store of the four 16x16 diagonal blocks of the inverse (fp32): block b at sD + b * DBLK, stride LDD.
constexpr int LDD = 20;
constexpr int DBLK = 16 * LDD;

// Column block J of Tm for blocks below the diagonal: X_iJ = -D_i sum_{k=J}^{i-1} A_ik X_kJ, X_JJ = D_J.
// A in sA (fp32, stride LF), the diagonal blocks D_i compact in sD (see LDD).  Blocks above the diagonal are zero.
template <typename T, int J, int LF, int LC>
__device__ __forceinline__ void tm_column(const float* sA, const float* sD, const f32x4& DJ, T* sTm) {
  f32x4 X[4];
  X[J] = DJ;
#pragma unroll
  for (int i = J + 1; i < 4; ++i) {
    f32x4 Y = zero4(), Xi = zero4();
#pragma unroll
    for (int k = J; k < i; ++k) mm16<T>(Y, ld_aslice<LF>(sA + 16 * i * LF + 16 * k), X[k]);
    mm16<T>(Xi, ld_aslice<LDD>(sD + i * DBLK), Y);
    X[i] = -Xi;
    put_tm_block<T, LC>(sTm, i, J, X[i]);
  }
#pragma unroll
  for (int i = 0; i < J; ++i) put_tm_block<T, LC>(sTm, i, J, zero4());
}

// Global accesses with the nontemporal hint (NT) stream past the caches' normal replacement: every kernel that
// reads an input once and writes each output once runs faster with it (measured per kernel; the reverse sweep,
// whose two V-block workgroups of a head share q, k, Tm and P through L2, keeps ordinary loads).
template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p) {
  if constexpr (NT) return __builtin_bit_cast(uint4, __builtin_nontemporal_load(static_cast<const u32x4*>(p)));
  else return *static_cast<const uint4*>(p);
}
template <bool NT>
__device__ __forceinline__ void st16(void* p, const uint4& v) {
  if constexpr (NT) __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), static_cast<u32x4*>(p));
  else *static_cast<uint4*>(p) = v;
}

// A ROWS x COLS tile of T held in registers as 16-byte vectors (ROWS*COLS*sizeof(T)/16 split over the NTH
// threads of a group; tid = thread index inside the group), used to prefetch the next chunk while the
// current one is computed.  The rows are read through a buffer resource whose range ends with the last valid
// row, so the hardware range check returns zeros for rows past the end of the sequence (no select, no access
// outside the valid rows); the per-lane offsets are 32-bit (the host keeps a chunk's row span of 64 * gld
// elements under 2 GiB).
template <typename T, int ROWS, int COLS, int NTH = NTHR, bool NT = false>
struct RegTile {
  static constexpr int E = 16 / sizeof(T);
  static constexpr int VPR = COLS / E;
  static constexpr int N = ROWS * VPR / NTH;
  static_assert(N * NTH == ROWS * VPR && N >= 1 && N <= 32, "tile must split evenly over the thread group");
  uint4 r[N];
  __device__ __forceinline__ void load(const T* g, int64_t gld, int valid, int tid) {
    const int nbytes = valid > 0 ? ((valid - 1) * (int)gld + COLS) * (int)sizeof(T) : 0;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(g), 0, nbytes, BUF_RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NTH, row = idx / VPR, c = (idx - row * VPR) * E;
      r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rs, (row * (int)gld + c) * (int)sizeof(T), 0, NT ? 2 : 0));
    }
  }
  __device__ __forceinline__ void store(T* s, int sld, int tid) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NTH, row = idx / VPR, c = (idx - row * VPR) * E;
      *reinterpret_cast<uint4*>(s + row * sld + c) = r[i];
    }
  }
  __device__ __forceinline__ void load(const T* g, int64_t gld, int valid) { load(g, gld, valid, threadIdx.x); }
  __device__ __forceinline__ void store(T* s, int sld) const { store(s, sld, threadIdx.x); }
};

// Per-token scalars (g, beta) of a chunk for the first wave: lanes past the end read token 0 instead (always in
// bounds) and report ok = false, so no wait for the data is forced at load time.
struct RegTok {
  float g, b;
  bool ok;
  __device__ __forceinline__ void load(const float* pg, const float* pb, int64_t row0, int64_t stride, int valid) {
    const int l = threadIdx.x & 63;
    ok = l < valid;
    const int64_t off = row0 + (ok ? l : 0) * stride;
    g = pg[off];
    b = pb ? pb[off] : 1.f;  // no beta: row scale 1
  }
};

// ---- fragment layout of the per-chunk [R][V] matrices in the workspace (states, R, their gradients) --------
// The sweeps hold S, R, dS and dR as MFMA accumulators and already form their permuted-k fragments (frag_acc2:
// element p of lane l is row 32 s + fragblk_row(l >> 4, p) of column 16 cb + (l & 15)).  Those fragments are
// stored as they are: block (s, cb) of an [R][V] matrix starts at element (s * V/16 + cb) * 512 and holds 8
// elements per lane, lane-contiguous, so each wave writes a block as one contiguous vector store per lane,
// with no staging.  The gradient kernel turns blocks back into row-major LDS tiles (FragTile).
__device__ __forceinline__ int fragblk_row(int g, int p) { return p < 4 ? 4 * g + p : 16 + 4 * g + (p - 4); }
template <typename T, bool NT = false>
__device__ __forceinline__ void store_fragblk(T* base, int rows, int s, int cb, int ncb,
                                              const typename Frag<T>::type& f) {
  // base: the chunk's [rows][16 ncb] matrix; bf16 blocks are written through a buffer resource over it
  const int e = ((s * ncb + cb) * 64 + lane_id()) * 8;
  if constexpr (sizeof(T) == 2) {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(base, 0, rows * ncb * 16 * 2, BUF_RSRC_WORD3);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f), rs, e * 2, 0, NT ? 2 : 0);
  } else {
    auto* p = reinterpret_cast<typename Frag<T>::type*>(base + e);
    if constexpr (NT) __builtin_nontemporal_store(f, p);
    else *p = f;
  }
}

// Columns [16 cb0, 16 cb0 + VS) of a fragment-layout [R][V] matrix (ncb = V / 16): loaded into registers as
// 8-element vectors by the NTH threads of the workgroup (tid = thread index), then written to a row-major LDS
// tile [R][ld] (column 0 = column 16 cb0).
template <typename T, int R, int VS, int NTH, bool NT = false>
struct FragTile {
  using F = typename Frag<T>::type;
  static constexpr int NVEC = R * VS / 8;
  static constexpr int N = (NVEC + NTH - 1) / NTH;
  static constexpr int NCBS = VS / 16;
  static_assert(R % 32 == 0 && VS % 16 == 0 && NVEC % 64 == 0, "whole fragment blocks only");
  F r[N];
  // base: the chunk's [R][16 ncb] matrix; bf16 reads go through a buffer resource over it (32-bit offsets).  With
  // live false (bf16 only) the resource's range is empty: the loads return zeros and fetch nothing, and the
  // instruction stream stays the same.
  __device__ __forceinline__ void load(const T* base, int ncb, int cb0, int tid, bool live = true) {
    [[maybe_unused]] const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(base), 0, live ? R * ncb * 16 * (int)sizeof(T) : 0, BUF_RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NTH;
      if (NVEC % NTH == 0 || idx < NVEC) {
        const int blk = idx >> 6, ln = idx & 63, s = blk / NCBS, cbl = blk - s * NCBS;
        const int e = ((s * ncb + cb0 + cbl) * 64 + ln) * 8;
        if constexpr (sizeof(T) == 2) {
          r[i] = __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b128(rs, e * 2, 0, NT ? 2 : 0));
        } else {
          const F* p = reinterpret_cast<const F*>(base + e);
          if constexpr (NT) r[i] = __builtin_nontemporal_load(p);
          else r[i] = *p;
        }
      }
    }
  }
  __device__ __forceinline__ void store(T* lds, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NTH;
      if (NVEC % NTH == 0 || idx < NVEC) {
        const int blk = idx >> 6, ln = idx & 63, s = blk / NCBS, cbl = blk - s * NCBS;
        T* dst = lds + (32 * s) * ld + 16 * cbl + (ln & 15);
#pragma unroll
        for (int p = 0; p < 8; ++p) dst[fragblk_row(ln >> 4, p) * ld] = r[i][p];
      }
    }
  }
  // sum over this thread's elements of r times the same elements of a column-major LDS tile laid out as store_t
  // writes one (bf16)
  __device__ __forceinline__ float dot_t(const T* lds, int ldt, int tid) const {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NTH;
      if (NVEC % NTH == 0 || idx < NVEC) {
        const int blk = idx >> 6, ln = idx & 63, s = blk / NCBS, cbl = blk - s * NCBS;
        const T* src = lds + (16 * cbl + (ln & 15)) * ldt + 32 * s + 4 * (ln >> 4);
        using V4 = typename std::conditional<sizeof(T) == 2, bf16x4, f32x4>::type;  // two 4-element runs
        const V4 a = *reinterpret_cast<const V4*>(src), b = *reinterpret_cast<const V4*>(src + 16);
#pragma unroll
        for (int p = 0; p < 4; p += 2) {
          acc = dot2(r[i][p], r[i][p + 1], a[p], a[p + 1], acc);
          acc = dot2(r[i][4 + p], r[i][5 + p], b[p], b[p + 1], acc);
        }
      }
    }
    return acc;
  }
  // Column-major LDS tile [VS][ldt] (element (row, col) at col * ldt + row): the lane's rows 4g..4g+3 and
  // 16+4g..16+4g+3 are two contiguous runs of 4, written as two vectors.  ldt must be a multiple of 4.
  __device__ __forceinline__ void store_t(T* lds, int ldt, int tid) const {
    using V4 = typename std::conditional<sizeof(T) == 2, bf16x4, f32x4>::type;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = tid + i * NTH;
      if (NVEC % NTH == 0 || idx < NVEC) {
        const int blk = idx >> 6, ln = idx & 63, s = blk / NCBS, cbl = blk - s * NCBS;
        T* dst = lds + (16 * cbl + (ln & 15)) * ldt + 32 * s + 4 * (ln >> 4);
        *reinterpret_cast<V4*>(dst) = V4{r[i][0], r[i][1], r[i][2], r[i][3]};
        *reinterpret_cast<V4*>(dst + 16) = V4{r[i][4], r[i][5], r[i][6], r[i][7]};
      }
    }
  }
};

// Copy a ROWS x COLS tile from LDS (stride sld) to global (row stride gld), 16-byte vectors, rows < valid only,
// by the NTH threads of the workgroup (tid = thread index).  The trip count is a compile-time constant and the
// stores are unconditional (a buffer resource over the valid rows drops the rest), so the compiler knows how
// many stores each thread has in flight and a later wait for an earlier load need not wait for these stores.
template <typename T, int ROWS, int COLS, int NTH = NTHR, bool NT = false>
__device__ __forceinline__ void s2g_rows(T* g, int64_t gld, const T* s, int sld, int valid, int tid = threadIdx.x) {
  constexpr int E = 16 / sizeof(T), VPR = COLS / E, NV = ROWS * VPR, N = (NV + NTH - 1) / NTH;
  static_assert(VPR * E == COLS, "whole 16-byte vectors per row");
  // 32-bit offsets, as for RegTile
  const int nbytes = valid > 0 ? ((valid - 1) * (int)gld + COLS) * (int)sizeof(T) : 0;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(g, 0, nbytes, BUF_RSRC_WORD3);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int idx = tid + i * NTH;
    if (NV % NTH == 0 || idx < NV) {
      const int r = idx / VPR, c = (idx - r * VPR) * E;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, *reinterpret_cast<const uint4*>(s + r * sld + c)),
                                             rs, (r * (int)gld + c) * (int)sizeof(T), 0, NT ? 2 : 0);
    }
  }
}

// ---- lower block-triangular 64 x 64 matrices (Tm, P) in HBM ----------------------------------------------------
// Only the blocks (bi, bj), bj <= bi, of 16 x 16 are stored, block bi (bi + 1) / 2 + bj of CH_TRI_ELEMS elements
// (5 KB instead of 8 KB in bf16); in LDS the matrices keep the full row-major layout, with the six blocks above the
// diagonal written as zeros once per workgroup.
// (row, first column) in the 64 x 64 matrix of 16-byte vector vi of the packed layout
template <typename T>
__device__ __forceinline__ void tri_vec_pos(int vi, int& row, int& col) {
  constexpr int E = 16 / sizeof(T), VPR = 16 / E, VPB = 16 * VPR;  // elements per vector; vectors per block row, block
  const int b = vi / VPB, wv = vi - b * VPB;
  const int bi = b >= 6 ? 3 : (b >= 3 ? 2 : (b >= 1 ? 1 : 0));
  const int rr = wv / VPR;
  row = 16 * bi + rr;
  col = 16 * (b - bi * (bi + 1) / 2) + (wv - rr * VPR) * E;
}

// A packed matrix held in registers as 16-byte vectors, to prefetch the next chunk's Tm or P as RegTile does.  The
// loads are unconditional -- threads past the last vector reload an earlier one and do not store it -- so the
// compiler counts the loads in flight exactly.
template <typename T, int NTH, bool NT>
struct TriTile {
  static constexpr int E = 16 / sizeof(T), NV = CH_TRI_ELEMS / E, N = (NV + NTH - 1) / NTH;
  static_assert(N * NTH <= 2 * NV, "a thread's spare vectors reload the first NV");
  uint4 r[N];
  __device__ __forceinline__ void load(const T* g, int tid) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int vi = tid + i * NTH;
      r[i] = ld16<NT>(g + (NV % NTH == 0 || vi < NV ? vi : vi - NV) * E);
    }
  }
  __device__ __forceinline__ void store(T* s, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int vi = tid + i * NTH;
      if (NV % NTH == 0 || vi < NV) {
        int row, col;
        tri_vec_pos<T>(vi, row, col);
        *reinterpret_cast<uint4*>(s + row * ld + col) = r[i];
      }
    }
  }
};

// The six zero blocks above the diagonal of a 64 x 64 LDS tile (ld elements per row), which packed stores never write
template <typename T, int NTH>
__device__ __forceinline__ void tri_zero_upper(T* s, int ld, int tid) {
  constexpr int E = 16 / sizeof(T), VPR = 16 / E, VPB = 16 * VPR;
  for (int vi = tid; vi < 6 * VPB; vi += NTH) {
    const int u = vi / VPB, wv = vi - u * VPB;  // upper block u: (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const int bi = u >= 5 ? 2 : (u >= 3 ? 1 : 0);
    const int bj = u + (bi == 0 ? 1 : (bi == 1 ? -1 : -2));
    const int rr = wv / VPR;
    *reinterpret_cast<uint4*>(s + (16 * bi + rr) * ld + 16 * bj + (wv - rr * VPR) * E) = make_uint4(0u, 0u, 0u, 0u);
  }
}

// Packed store of the lower blocks of a 64 x 64 LDS tile (ld elements per row) to global memory
template <typename T, int NTH, bool NT>
__device__ __forceinline__ void s2g_tri(T* g, const T* s, int ld, int tid) {
  constexpr int E = 16 / sizeof(T), NV = CH_TRI_ELEMS / E, N = (NV + NTH - 1) / NTH;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int vi = tid + i * NTH;
    if (NV % NTH == 0 || vi < NV) {
      int row, col;
      tri_vec_pos<T>(vi, row, col);
      st16<NT>(g + vi * E, *reinterpret_cast<const uint4*>(s + row * ld + col));
    }
  }
}

// The elements of a row-major LDS tile at this lane's accumulator positions of output tile (rows r0.., columns
// c0..): rows r0 + 4 (l >> 4) + i (i = 0..3) of column c0 + (l & 15).  bf16: one transposing read.
template <typename T>
__device__ __forceinline__ void acc_vals(const T* p, int ld, int r0, int c0, float (&v)[4], int l = lane_id()) {
  if constexpr (sizeof(T) == 2) {
    const bf16x4 t = ld_tr4(p, ld, c0, r0 + 4 * (l >> 4), l);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = to_f(t[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = p[(r0 + acc_row(i, l)) * ld + c0 + acc_col(l)];
  }
}

// Four consecutive elements p[c * ld + r0 .. r0 + 3] of a tile stored with r contiguous (one 8-byte read in bf16,
// 16 bytes in fp32; r0 a multiple of 4 and c * ld * sizeof(T) a multiple of 8 or 16): the accumulator positions
// of this lane in a column-major tile.
template <typename T>
__device__ __forceinline__ void run4(const T* p, int ld, int c, int r0, float (&v)[4]) {
  if constexpr (sizeof(T) == 2) {
    const bf16x4 t = *reinterpret_cast<const bf16x4*>(p + c * ld + r0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = to_f(t[i]);
  } else {
    const f32x4 t = *reinterpret_cast<const f32x4*>(p + c * ld + r0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = t[i];
  }
}

// ---- chunk factors, in three barrier-separated phases ------------------------------------------------------
// Each phase is a separate function; the caller places the barriers between them.
//
// factors_kq: K U^T and Q U^T on MFMA (row block = wave), then
//   A_ij = beta_i (K U^T)_ij exp(G_i - G_j) (i > j) -> sA  (fp32, strict lower)
//   P_ij = s (Q U^T)_ij exp(G_i - G_j) (i >= j)     -> sP  (PMODE 1, row-major; PMODE 0: none, sQ unused)
// U is the write key (U = K for the gated delta rule).  Inputs: sK, sU (and sQ) rows of the chunk, zero past the
// sequence end; sG (cumulative log-decay); sB (row scale beta, zero past the end).  Wave w reads only rows
// 16w..16w+15 of sK and sQ and writes only the same rows of sA and sP, and its K and Q fragments are all read
// before its first write, so sA may share memory with sQ row for row (same row pitch in bytes).
template <typename T, int K, int PMODE>
__device__ __forceinline__ void factors_kq(const T* sK, const T* sU, const T* sQ, const float* sG, const float* sB,
                                           float scale, float* sA, T* sP, int w) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LF = CH + 4;
  // masks are selects on values computed unconditionally (exp of min(G_i - G_j, 0) cannot overflow), so the
  // epilogue has no branches around its LDS reads
  float Gr[4], Br[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    Gr[i] = sG[16 * w + acc_row(i)];
    Br[i] = sB[16 * w + acc_row(i)];
  }
  // the row block's K (and Q) fragments are read once; each column block's U fragment serves both products
  typename Frag<T>::type ak[K / 32], aq[K / 32];
#pragma unroll
  for (int s = 0; s < K / 32; ++s) {
    ak[s] = frag_kc(sK, LK, 16 * w, 32 * s);
    if constexpr (PMODE != 0) aq[s] = frag_kc(sQ, LK, 16 * w, 32 * s);
  }
  asm volatile("" ::: "memory");  // the reads above stay ahead of the sA writes below (sA may overlay sQ)
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < K / 32; ++s) {
      const auto bk = frag_kc(sU, LK, 16 * n, 32 * s);
      mma(kk, ak[s], bk);
      if constexpr (PMODE != 0) mma(qk, aq[s], bk);
    }
    const int cc = 16 * n + acc_col();
    const float Gc = sG[cc];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + acc_row(i);
      const float e = __expf(fminf(Gr[i] - Gc, 0.f));
      sA[r * LF + cc] = r > cc ? Br[i] * kk[i] * e : 0.f;
      if constexpr (PMODE == 1) sP[r * LC + cc] = from_f<T>(r >= cc ? scale * qk[i] * e : 0.f);
    }
  }
}

// factors_diag (after factors_kq; it reads only the row block of A that the same wave wrote, so no barrier is
// needed in between): wave w inverts diagonal block w of I + A, writes it to sD and to its Tm block (row-major) and
// returns it for factors_merge.
template <typename T>
__device__ __forceinline__ f32x4 factors_diag(const float* sA, float* sD, T* sTm, int w) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LC = CH + PT, LF = CH + 4;
  const f32x4 D = inv_diag16<T, LF>(sA + 16 * w * LF + 16 * w);
#pragma unroll
  for (int i = 0; i < 4; ++i) sD[w * DBLK + acc_row(i) * LDD + acc_col()] = D[i];
  put_tm_block<T, LC>(sTm, w, w, D);
  return D;
}

// factors_merge (after a barrier following factors_diag): the blocks of Tm below the diagonal, column block =
// wave w, straight into sTm.  Tm is complete once every wave has returned (caller's barrier).
template <typename T>
__device__ __forceinline__ void factors_merge(const f32x4& D, const float* sA, const float* sD, T* sTm, int w) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LC = CH + PT, LF = CH + 4;
  switch (w) {
    case 0: tm_column<T, 0, LF, LC>(sA, sD, D, sTm); break;
    case 1: tm_column<T, 1, LF, LC>(sA, sD, D, sTm); break;
    case 2: tm_column<T, 2, LF, LC>(sA, sD, D, sTm); break;
    default: tm_column<T, 3, LF, LC>(sA, sD, D, sTm); break;
  }
}

}  // namespace gdn
