// Chunkwise gated delta rule, backward.
//
// The backward takes the chunk factors (Tm, P, G), R and the state entering every chunk (every second one:
// state_stride) from the stashing forward, or rebuilds them first (chunk factors kernel, then the forward sweep in recompute mode), then runs:
//
// bwd_state: one workgroup per (V block of 64 columns, or 32 when the grid fits the device, b*h), reverse over
//   chunks, reading the chunk factors; each wave carries a 16-column slab of dS in MFMA accumulators.
//     dR  = P^T dO + Kd dS_C                         Kd = diag(exp(G_C - G)) K
//     dY  = Tm^T dR                                  (the gradient w.r.t. Y, where R = Tm Y, Y = beta (V - gamma K S0))
//     dS0 = gamma_C dS_C + s (diag(gamma) Q)^T dO - K^T diag(beta gamma) dY
//   Writes dS_C (the gradient w.r.t. the state leaving each chunk) and dY per chunk, and dh0.
//   (The reverse state-gradient recurrence of fla's chunk_gated_delta_rule_bwd_dhu, called at
//   archbench/layers/nsgdn.py:378.)
//
// bwd_intra: persistent, one workgroup per CU looping over (chunk, b*h) items with the full K and V of a chunk;
// all gradients.  With R = Tm Y the WY backward needs no Tm: dA = -Tm^T (dR Y^T) Tm^T = -(Tm^T dR)(Tm Y)^T =
// -dY R^T, and the gradient through Y's K S0 term is -beta gamma dY S0^T, so
//     dq  = s gamma (dO S0^T) + (dP o sE) K                         dP = dO R^T  (i >= j)
//     dk  = dte (R dS_C^T) + (dP o sE)^T Q - beta gamma (dY S0^T) + (D + D^T) K
//     dv  = beta dY                                                 dA = -dY R^T (strict lower), D = dA o beta_i E
//     dbeta = -gamma (dY S0^T . k) + (dY . v) + rowsum(dA o KK o E)
//     dG  = s gamma (dO S0^T . q) - dte (R dS_C^T . k) - beta gamma (dY S0^T . k)
//           + rowsum - colsum of (dP o P + dA o A),   dG_last += sum dte (R dS_C^T . k) + gamma_C <dS_C, S0>
//     dg  = reverse chunk-local cumsum of dG
//   (fla's chunk_bwd_dv_local + chunk_bwd_dqkwg, the WY backward of nsgdn.py:279-330 and the reverse cumsum
//   of nsgdn.py:381, fused per chunk.)  Reductions are deterministic: no atomics anywhere.
//
// SEPU (separate write keys U, the n-step family's nsgdn_chunk_bwd, nsgdn.py:369-382): U replaces K wherever K
// is a write key -- Kd dS_C in dR, the column side of K K^T and Q K^T, and the state update -- and the
// gradients split into dk (read: -beta gamma dY S0^T + D U) and du (write: dte R dS_C^T + (dP o sE)^T Q + D^T K);
// beta may be absent (row scale 1, no dbeta).
#include "gdn_chunk_common.h"
#include "gdn_launch.h"

namespace gdn {

// Two waves per 16-column slab of the V block (BV / 16 slabs: eight waves for BV = 64, four for BV = 32): waves
// w and w + NSL share the slab 16 (w % NSL) of dS.  Half hf = w / NSL holds rows 64 hf .. of dS (K = 128; rows
// K/2 hf .. in general) and computes dR and Z for the chunk's token rows 32 hf .. 32 hf + 31.  Per chunk the
// halves swap through LDS: the partial K dS of the other half's token rows (fp32), then the dR fragments, then
// the Z fragments (16 bytes per lane each).
template <int BV>
constexpr int state_threads() { return 128 * (BV / 16); }
// the two V-block workgroups of a head read the same q, k, Tm and P (the second from L2): ordinary loads; dS_C and
// dR are written once, nontemporal
constexpr bool STATE_NT_LOAD = false, STATE_NT_STORE = true;
constexpr bool INTRA_NT = true;  // every read and write of the gradient kernel is single-use

// STORE: write dS_C and dY for every chunk (the gradient kernel reads them); without it (the local pass of a
// segmented sweep) only dh0 is written.
template <typename T, int K, int BV, bool SEPU, bool STORE>
__global__ __launch_bounds__(state_threads<BV>()) __attribute__((amdgpu_waves_per_eu(2))) void bwd_state_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ u, const T* __restrict__ dout,
    const float* __restrict__ beta,
    const T* __restrict__ gTm, const T* __restrict__ gP, const float* __restrict__ gGc,
    const float* __restrict__ dhT, float* __restrict__ dh0, T* __restrict__ wsdH, T* __restrict__ wsdY, int T_,
    int H, int V, int NT, float scale, int ns) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LV = BV + PT;
  constexpr int NKH = K / 32;     // row tiles of dS per half
  constexpr int NSH = K / 64;     // 32-row fragments of dS per half
  constexpr int NSL = BV / 16, SW = 2 * NSL, STH = 64 * SW;  // slabs, waves, threads
  static_assert(NSL == 2 || NSL == 4, "a wave pair per 16-column slab, two or four slabs");
  using F = typename Frag<T>::type;
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];
  __shared__ __attribute__((aligned(16))) T sU_[SEPU ? CH * LK : 8];
  T* sU = SEPU ? sU_ : sK;  // write keys
  __shared__ __attribute__((aligned(16))) T sQ[CH * LK];
  __shared__ __attribute__((aligned(16))) T sdO[CH * LV];  // dO rows of this V block
  __shared__ __attribute__((aligned(16))) T sTm[CH * LC];
  __shared__ __attribute__((aligned(16))) T sP[CH * LC];
  __shared__ __attribute__((aligned(16))) f32x4 xKd[SW][2][64];      // partial K dS for the other half's rows
  __shared__ __attribute__((aligned(16))) F xR[SW][64], xZ[SW][64];  // dR and Z fragments
  // per token: exp(G), exp(G_C - G) and -beta exp(G) (formed once per chunk by the first wave)
  __shared__ float sGam[CH], sDte[CH], sBGn[CH];

  int vb, bh;
  sweep_block(V / BV, gridDim.x * BV / V, vb, bh);
  const int b = bh / H, h = bh - b * H;
  const int seg = b % ns;  // segment of sequence b / ns (ns = 1: not segmented)
  // The local pass of a segmented sweep (STORE = false) skips each sequence's first segment (its entering-state
  // gradient is the main sweep's dh0) and starts the last from the sequence's dhT, so that its result already
  // carries dhT.  dh0: per swept sequence in the local pass; otherwise, when segmented, only from the first
  // segment of each sequence, at the sequence's index.  dhT: per swept sequence in the main pass.
  if (!STORE && seg == 0) return;  // uniform over the workgroup, before any barrier
  const bool put_dh0 = !STORE || seg == 0;
  const int64_t dh0_base = (!STORE ? (int64_t)bh : (int64_t)(b / ns) * H + h) * K * V;
  const bool use_dhT = dhT && (STORE || seg == ns - 1);
  const int64_t dhT_base = (STORE ? (int64_t)bh : (int64_t)(b / ns) * H + h) * K * V;
  const int v0 = vb * BV;
  const int w = wave_id(), l = lane_id();
  const int ws = w & (NSL - 1), hf = w / NSL;  // column slab; half of dS's rows and of the chunk's tokens
  const int c0 = 16 * ws;
  const int ncb = V / 16, cb = vb * (BV / 16) + ws;  // fragment-layout column block of the slab
  const int k0 = (K / 2) * hf;                       // first dS row of this half
  const int tid = threadIdx.x;
  auto row0_of = [&](int c) { return ((int64_t)b * T_ + (int64_t)c * CH) * H + h; };
  auto nvalid_of = [&](int c) { return min(CH, T_ - c * CH); };

  RegTile<T, CH, K, STH, STATE_NT_LOAD> rk, rq, ru;
  RegTile<T, CH, BV, STH, STATE_NT_LOAD> rdo;
  TriTile<T, STH, STATE_NT_LOAD> rtm, rp;  // packed lower blocks
  float pG = 0.f, pB = 0.f;
  // The next chunk's reads go out in three batches (k, q after the first barrier, dO after the second; Tm, P,
  // G, beta after the dR exchange), so that no wave stalls on a full memory queue for the whole set at once
  // (three batches measured 2% faster than two).
  auto prefetch = [&](int c, int part) {
    const int64_t row0 = row0_of(c);
    const int nv = nvalid_of(c);
    if (part != 2) {
      rk.load(k + row0 * K, (int64_t)H * K, nv, tid);
      if constexpr (SEPU) ru.load(u + row0 * K, (int64_t)H * K, nv, tid);
      rq.load(q + row0 * K, (int64_t)H * K, nv, tid);
    }
    if (part != 1) {
      rdo.load(dout + row0 * V + v0, (int64_t)H * V, nv, tid);
    }
  };
  auto prefetch2 = [&](int c) {
    const int64_t row0 = row0_of(c), cidx = (int64_t)bh * NT + c;
    const int nv = nvalid_of(c);
    rtm.load(gTm + cidx * CH_TRI_ELEMS, tid);
    rp.load(gP + cidx * CH_TRI_ELEMS, tid);
    if (w == 0) {
      pG = gGc[cidx * CH + l];
      pB = l < nv ? (beta ? beta[row0 + (int64_t)l * H] : 1.f) : 0.f;
    }
  };

  f32x4 dS[NKH];
#pragma unroll
  for (int t = 0; t < NKH; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dS[t][i] = use_dhT ? dhT[dhT_base + (int64_t)(k0 + 16 * t + acc_row(i)) * V + v0 + c0 + acc_col()] : 0.f;

  auto chunk = [&](int c) {
    const int64_t cidx = (int64_t)bh * NT + c;
    rk.store(sK, LK, tid);
    if constexpr (SEPU) ru.store(sU, LK, tid);
    rq.store(sQ, LK, tid);
    rdo.store(sdO, LV, tid);
    rtm.store(sTm, LC, tid);
    rp.store(sP, LC, tid);
    if (w == 0) {
      const float gam = __expf(pG), GCl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pG), CH - 1));
      sDte[l] = __expf(GCl - pG);
      sGam[l] = gam;
      sBGn[l] = -pB * gam;
    }
    __syncthreads();
    if (c > 0) prefetch(c - 1, 1);

    // dS leaving the chunk -> dh (fragment layout); partial U dS over this half's rows, for all tokens
    F dSb[NSH];
#pragma unroll
    for (int s = 0; s < NSH; ++s) {
      dSb[s] = frag_acc2<T>(dS[2 * s], dS[2 * s + 1]);
      if constexpr (STORE) store_fragblk<T, STATE_NT_STORE>(wsdH + cidx * K * V, K, NSH * hf + s, cb, ncb, dSb[s]);
    }
    // kd[j]: this half's token rows 32 hf + 16 j (first), kd[2 + j]: the other half's (to the partner); the rows
    // are chosen by address, so no value is selected by the half
    const int tmine = 32 * hf, tother = 32 - tmine;  // first token of each half
    f32x4 kd[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      kd[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int r0 = (jj < 2 ? tmine : tother) + 16 * (jj & 1);
#pragma unroll
      for (int s = 0; s < NSH; ++s) mma(kd[jj], frag_kc_perm(sU, LK, r0, k0 + 32 * s), dSb[s]);
    }
    xKd[w][0][l] = kd[2];
    xKd[w][1][l] = kd[3];
    F dOb[2], dOg[2];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      dOb[ib] = frag_oct(sdO, LV, c0, 32 * ib);
#pragma unroll
      for (int e = 0; e < 8; ++e) dOg[ib][e] = from_f<T>(to_f(dOb[ib][e]) * sGam[32 * ib + 8 * (l >> 4) + e]);
    }
    __syncthreads();
    if (c > 0) prefetch(c - 1, 2);
    // dR (this half's token rows) = diag(exp(G_C - G)) K dS + P^T dO
    f32x4 dR[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rt_ = 2 * hf + j;
      const f32x4 mine = kd[j];
      const f32x4 other = xKd[w ^ NSL][j][l];
#pragma unroll
      for (int i = 0; i < 4; ++i) dR[j][i] = sDte[16 * rt_ + acc_row(i)] * (mine[i] + other[i]);
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) mma(dR[j], frag_oct(sP, LC, 16 * rt_, 32 * ib), dOb[ib]);
    }
    // dR to the other half; dY (this half's token rows) = Tm^T dR -> global; Z = -diag(beta gamma) dY
    const F dRmine = frag_acc2<T>(dR[0], dR[1]);
    xR[w][l] = dRmine;
    __syncthreads();
    if (c > 0) prefetch2(c - 1);
    const F dRother = xR[w ^ NSL][l];
    f32x4 Z[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rt_ = 2 * hf + j;
      Z[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma(Z[j], frag_oct_perm(sTm, LC, 16 * rt_, tmine), dRmine);
      mma(Z[j], frag_oct_perm(sTm, LC, 16 * rt_, tother), dRother);
    }
    if constexpr (STORE)
      store_fragblk<T, STATE_NT_STORE>(wsdY + cidx * CH * V, CH, hf, cb, ncb, frag_acc2<T>(Z[0], Z[1]));
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        Z[j][i] *= sBGn[16 * (2 * hf + j) + acc_row(i)];
      }
    const F Zmine = frag_acc2<T>(Z[0], Z[1]);
    xZ[w][l] = Zmine;
    __syncthreads();
    const F Zother = xZ[w ^ NSL][l];
    // this half's rows of dS <- gamma_C dS + K^T Z (accumulated in place) + s Q^T (gamma dO)
    const float gC = sGam[CH - 1];  // exp(G_C)
#pragma unroll
    for (int t = 0; t < NKH; ++t) {
      f32x4 a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) mma(a1, frag_oct(sQ, LK, k0 + 16 * t, 32 * ib), dOg[ib]);
      dS[t] *= gC;
      mma(dS[t], frag_oct_perm(sK, LK, k0 + 16 * t, tmine), Zmine);
      mma(dS[t], frag_oct_perm(sK, LK, k0 + 16 * t, tother), Zother);
      dS[t] += scale * a1;
    }
    __syncthreads();  // every wave done with this chunk's inputs
  };
  // the blocks of Tm and P above the diagonal stay zero (the packed loads write the others); ordered before any
  // read by the first chunk's first barrier
  tri_zero_upper<T, STH>(sTm, LC, tid);
  tri_zero_upper<T, STH>(sP, LC, tid);
  prefetch(NT - 1, 0);
  prefetch2(NT - 1);
  for (int c = NT - 1; c >= 0; --c) chunk(c);
  if (dh0 && put_dh0) {
#pragma unroll
    for (int t = 0; t < NKH; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dh0[dh0_base + (int64_t)(k0 + 16 * t + acc_row(i)) * V + v0 + c0 + acc_col()] = dS[t][i];
  }
}

// ---------------------------------------------------------------------------------------------------------
// One reduce-scatter round over a 16-lane DPP row: values a[0 .. 2N) -> a[0 .. N).  The lane whose bit `hi` is
// clear keeps a[k] and sends a[k + N], its partner (DPP pattern CTRL, which pairs lanes with opposite bits)
// the reverse; each keeps its value plus the one it receives.
template <int N, int CTRL>
__device__ __forceinline__ void rs_round(float* a, int hi) {
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float keep = hi ? a[k + N] : a[k], send = hi ? a[k] : a[k + N];
    a[k] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), CTRL, 0xf, 0xf, true));
  }
}

// Sum of the 4 rows a lane holds plus the other 3 lane groups: the per-column sum of a 16x16 tile.
__device__ __forceinline__ float colsum_tile(const f32x4& x) {
  return xor32_sum(xor16_sum(x[0] + x[1] + x[2] + x[3]));
}

// Eight waves, two per SIMD: wave w owns row block rb = w & 3 (16 tokens of the chunk) and half hf = w >> 2 of
// the output column tiles of every product; per-row reductions add the two halves through LDS.
constexpr int IW = 2 * NWAVE;  // waves of the intra kernel
constexpr int ITH = IW * 64;   // its threads

template <typename T, int K, int V, int VS, bool SEPU, bool HALF>
__global__ __launch_bounds__(ITH) void bwd_intra_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ u, const T* __restrict__ v,
    const float* __restrict__ beta, const T* __restrict__ dout, const float* __restrict__ wsGc,
    const T* __restrict__ wsH, const T* __restrict__ wsR, const T* __restrict__ wsdH, const T* __restrict__ wsdY,
    T* __restrict__ dq, T* __restrict__ dk, T* __restrict__ du, T* __restrict__ dv, float* __restrict__ dg,
    float* __restrict__ dbeta, int T_, int H, int NT, int BH, float scale) {
  constexpr int PT = 16 / sizeof(T);
  constexpr int LK = K + PT, LC = CH + PT, LS = VS + PT;
  constexpr int NKT = K / 16;   // column tiles over K
  constexpr int NVT = VS / 16;  // column tiles over a V slab
  constexpr int HK = NKT / 2, HV = NVT / 2, HC = 2;  // tiles per half: over K, over the slab, over the chunk
  // slab region: V phase {dO, V : CH x LS; R^T, dY^T : VS x LC; S0^T, dSC^T : VS x LK (column-major, so the
  // fragment-layout tiles are written as 4-element runs)}; K phase {dq, dk staging : CH x LK; D, dPm : CH x LC}
  constexpr int SLAB_V = 2 * CH * LS + 2 * VS * LC + 2 * VS * LK;
  constexpr int SLAB_K = 2 * CH * LK + 2 * CH * LC;
  constexpr int SLAB = SLAB_V > SLAB_K ? SLAB_V : SLAB_K;
  __shared__ __attribute__((aligned(16))) T sQ[CH * LK];
  __shared__ __attribute__((aligned(16))) T sK[CH * LK];
  __shared__ __attribute__((aligned(16))) T sU_[SEPU ? CH * LK : 8];
  T* sU = SEPU ? sU_ : sK;  // write keys
  __shared__ __attribute__((aligned(16))) T slab[SLAB];
  __shared__ __attribute__((aligned(16))) T sdv[CH * LS];  // dv of the current slab, for the coalesced store
  __shared__ float sG[CH], sB[CH], sdG[CH], sLast[CH], sColZ[NWAVE][CH], sRed[IW];
  __shared__ float sGam[CH], sDte[CH];  // exp(G) and exp(G_C - G) per token (formed once per chunk by wave 0)
  __shared__ float sRow[2][6][CH];  // per-half row sums: rq, rk, dbV, rx, dbA, rz
  // HALF (state stride 2): the stash holds the state entering even chunks only; an even chunk advances it through
  // itself into sS1t (the odd chunk's entering state, S1^T [V][LK]) with exp(G_C - G) per row from sDte
  static_assert(!HALF || (sizeof(T) == 2 && !SEPU), "state stride 2: bf16 without separate write keys");
  __shared__ __attribute__((aligned(16))) T sS1t[HALF ? V * LK : 8];

  T* sdO = slab;
  T* sV = sdO + CH * LS;
  T* sRt = sV + CH * LS;      // R^T     [VS][LC]
  T* sdYt = sRt + VS * LC;    // dY^T    [VS][LC]
  T* sS0t = sdYt + VS * LC;   // S0^T    [VS][LK]
  T* sdSCt = sS0t + VS * LK;  // dS_C^T  [VS][LK]

  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int rb = w & (NWAVE - 1), hf = w >> 2;
  // work items: chunks, or (HALF) pairs of chunks (2 j, 2 j + 1) of one sequence, the second if it exists
  const int NT2 = HALF ? (NT + 1) / 2 : NT;
  const int nitem = BH * NT2;
  // items in chunk-position-major order (item = position * BH + b*h): the workgroups in flight together read the
  // same token rows of every head, so each row of q, k, v and dO is fetched by all its heads at about the same time
  auto item_chunk = [&](int it) {  // the first chunk of work item it
    const int pos = (int)((unsigned)it / (unsigned)BH), bh_ = it - pos * BH;
    return bh_ * NT + (HALF ? 2 * pos : pos);
  };
  auto chunk_pos = [&](int ci_) { return ci_ - (int)((unsigned)ci_ / (unsigned)NT) * NT; };  // chunk in sequence
  // the stash slot of chunk ci's entering state (HALF: even chunks only)
  auto state_slot = [&](int ci_) -> int64_t {
    if constexpr (HALF) {
      const int bh_ = (int)((unsigned)ci_ / (unsigned)NT);
      return (int64_t)bh_ * NT2 + (ci_ - bh_ * NT) / 2;
    } else {
      return ci_;
    }
  };
  // thread index and lane, re-derived opaquely in every chunk iteration (see the lane-dependent helpers)
  int tid = threadIdx.x, l = tid & 63;

  // Chunk ci = bh NT + c (also its index in the workspace): first row in the token-major tensors, valid rows.
  auto chunk_rows = [&](int ci, int& nv) -> int64_t {
    const int bh = (int)((unsigned)ci / (unsigned)NT), c = ci - bh * NT;
    const int b = bh / H, h = bh - b * H;
    nv = min(CH, T_ - c * CH);
    return ((int64_t)b * T_ + c * CH) * H + h;
  };

  // Global reads are issued as 16-byte register tiles (RegTile, FragTile) in the order they are consumed, each
  // V slab in two groups: A = {dO, V, R, dY} (and G, beta first) feeds dO R^T, dY R^T and dv; B = {S0, dS_C}
  // feeds the products with the states.  Group B and Q, K stay in flight while group A is computed, and the
  // next slab's groups are issued as soon as their registers are free.
  RegTile<T, CH, K, ITH, INTRA_NT> tq, tk, tu;
  RegTile<T, CH, VS, ITH, INTRA_NT> rdo, rv;
  FragTile<T, CH, VS, ITH, INTRA_NT> rr, rdy;
  FragTile<T, K, VS, ITH, INTRA_NT> rs0, rdsc;
  auto load_a = [&](int64_t ci, int64_t r0, int nv, int vs) {
    rdo.load(dout + r0 * V + vs, (int64_t)H * V, nv, tid);
    rv.load(v + r0 * V + vs, (int64_t)H * V, nv, tid);
    rr.load(wsR + ci * CH * V, V / 16, vs / 16, tid);
    rdy.load(wsdY + ci * CH * V, V / 16, vs / 16, tid);
  };
  // group B: the entering state (not read for the odd chunk of a HALF pair: s0 false) and the leaving state's
  // gradient
  auto load_b = [&](int64_t ci, int vs, bool s0) {
    rs0.load(wsH + state_slot((int)ci) * K * V, V / 16, vs / 16, tid, s0);
    rdsc.load(wsdH + ci * K * V, V / 16, vs / 16, tid);
  };
  // The reads a chunk needs first: G, beta and the first slab's groups.  The workgroups are persistent (one per
  // CU, looping over chunks) and issue these for their next chunk during the current chunk's K phase, which reads
  // no global memory: the loads are served while the K phase computes (group A at the K phase's start, group B
  // after its first barrier: issued together, the waves stalled on the memory queue instead of computing).
  float pg, pb;
  auto is_odd = [&](int ci_) { return HALF && (chunk_pos(ci_) & 1); };
  auto load_first = [&](int ci, bool order, bool with_b) {
    int nv;
    const int64_t r0 = chunk_rows(ci, nv);
    pg = wsGc[(int64_t)ci * CH + (tid & (CH - 1))];
    pb = beta ? beta[r0 + (int64_t)((tid & (CH - 1)) < nv ? (tid & (CH - 1)) : 0) * H] : 1.f;
    load_a(ci, r0, nv, 0);
    if (order) {
      // A bare barrier (no fence: nothing waits for the loads) so that every wave has issued group A before any
      // wave issues group B, Q and K.  The memory path serves a CU's loads roughly in issue order and the older
      // waves issue first, so without it the second wave of each SIMD gets its group A behind the first waves'
      // B, Q and K, and the first barrier waits for nearly all of the chunk's first reads.
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (with_b) load_b(ci, 0, !is_odd(ci));
  };
  if ((int)blockIdx.x < nitem) load_first(item_chunk(blockIdx.x), true, true);

#pragma unroll 1
  for (int it = blockIdx.x, ci = item_chunk(it); it < nitem;) {
  asm volatile("" : "+v"(tid));
  l = tid & 63;
  int nvalid;
  const int64_t row0 = chunk_rows(ci, nvalid);
  const int64_t cidx = ci;
  // HALF: odd chunks take their entering state from sS1t; an even chunk with an odd partner fills it
  const bool odd = is_odd(ci);
  const bool advance = HALF && !odd && chunk_pos(ci) + 1 < NT;
  // the next chunk: this pair's odd one, else the next item's first (or this chunk again after the last item:
  // the prefetch stays unconditional)
  const bool in_pair = advance;
  const int it_next = in_pair ? it : it + (int)gridDim.x;
  const int cnext = in_pair ? ci + 1 : (it_next < nitem ? item_chunk(it_next) : ci);
  tq.load(q + row0 * K, (int64_t)H * K, nvalid, tid);
  tk.load(k + row0 * K, (int64_t)H * K, nvalid, tid);
  if constexpr (SEPU) tu.load(u + row0 * K, (int64_t)H * K, nvalid, tid);
  if (tid < CH) {
    sG[tid] = pg;
    sB[tid] = tid < nvalid ? pb : 0.f;
    const float gl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pg), CH - 1));  // G_C (wave 0)
    sGam[tid] = __expf(pg);
    sDte[tid] = __expf(gl - pg);
  }

  // ---- V phase: contractions over V, slab by slab -------------------------------------------------------
  // column tile j of this wave: n = HC*hf + j over the chunk, HK*hf + j over K, HV*hf + j over the slab
  f32x4 aP[HC], aDA[HC], aQg[HK], aKd[HK], aKY[HK];
#pragma unroll
  for (int j = 0; j < HC; ++j) aP[j] = aDA[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < HK; ++j) aQg[j] = aKd[j] = aKY[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float dbV[4] = {0.f, 0.f, 0.f, 0.f};
  float sdot = 0.f;  // partial <dS_C, S0>
  typename Frag<T>::type adv_a[2];  // HALF: the state advance's first operand, formed in the first slab

  // Unrolled up to two slabs: with the slab tests resolved at compile time the compiler counts the loads in
  // flight exactly (four slabs unrolled would spill).
  constexpr int SLAB_UNROLL = V / VS <= 2 ? V / VS : 1;
#pragma unroll SLAB_UNROLL
  for (int vs = 0; vs < V; vs += VS) {
    // group A: dO R^T, dY R^T; dv = beta dY and dbeta += dY . v
    rdo.store(sdO, LS, tid);
    rv.store(sV, LS, tid);
    rr.store_t(sRt, LC, tid);
    rdy.store_t(sdYt, LC, tid);
    __syncthreads();
    if (vs + VS < V) load_a(cidx, row0, nvalid, vs + VS);
#pragma unroll
    for (int j = 0; j < HC; ++j) {
      const int n = HC * hf + j;
      mma_blk<true, false, VS>(aP[j], sdO, LS, 16 * rb, sRt, LC, 16 * n, l);
      mma_blk<false, false, VS>(aDA[j], sdYt, LC, 16 * rb, sRt, LC, 16 * n, l);
    }
#pragma unroll
    for (int j = 0; j < HV; ++j) {
      const int vc = 16 * (HV * hf + j) + acc_col(l), r0 = 16 * rb + 4 * (l >> 4);
      float dy[4], vv[4];
      run4(sdYt, LC, vc, r0, dy);
      acc_vals(sV, LS, 16 * rb, 16 * (HV * hf + j), vv, l);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dbV[i] += dy[i] * vv[i];
        sdv[(r0 + i) * LS + vc] = from_f<T>(sB[r0 + i] * dy[i]);
      }
    }
    // group B: dO S0^T, R dS_C^T, dY S0^T, <dS_C, S0> (the last from the registers: each thread holds the same
    // elements of both tiles)
    rdsc.store_t(sdSCt, LK, tid);
    if (HALF && odd) {  // the entering state is the even chunk's advance in sS1t (rs0 loaded nothing)
      sdot += rdsc.dot_t(sS1t + vs * LK, LK, tid);
    } else {
      rs0.store_t(sS0t, LK, tid);
#pragma unroll
      for (int i = 0; i < decltype(rs0)::N; ++i)
        if (decltype(rs0)::NVEC % ITH == 0 || tid + i * ITH < decltype(rs0)::NVEC)  // loaded by this thread
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            sdot = dot2(rdsc.r[i][e], rdsc.r[i][e + 1], rs0.r[i][e], rs0.r[i][e + 1], sdot);
    }
    if (vs == 0) {
      tq.store(sQ, LK, tid);
      tk.store(sK, LK, tid);
      if constexpr (SEPU) tu.store(sU, LK, tid);
    }
    __syncthreads();
    if (vs + VS < V) load_b(cidx, vs + VS, !odd);
    s2g_rows<T, CH, VS, ITH, INTRA_NT>(dv + row0 * V + vs, (int64_t)H * V, sdv, LS, nvalid, tid);
    const T* s0t = HALF && odd ? sS1t + vs * LK : sS0t;  // S0^T of this slab
#pragma unroll
    for (int j = 0; j < HK; ++j) {
      const int n = HK * hf + j;
      mma_blk<true, false, VS>(aQg[j], sdO, LS, 16 * rb, s0t, LK, 16 * n, l);
      mma_blk<false, false, VS>(aKd[j], sRt, LC, 16 * rb, sdSCt, LK, 16 * n, l);
      mma_blk<false, false, VS>(aKY[j], sdYt, LC, 16 * rb, s0t, LK, 16 * n, l);
    }
    if constexpr (HALF) {
      if (advance) {
        // S1 = gamma_C S0 + (diag(exp(G_C - G)) K)^T R over this slab's columns, the odd chunk's entering state
        // (the forward sweep's update, nsgdn.py:240-249): [K] x [VS] in 16 x 16 tiles, wave w taking NA tiles of
        // one row tile so that one A operand serves them all; S1^T to sS1t in the column-major layout of sS0t
        constexpr int NA = NKT * NVT / IW;
        static_assert(NA >= 1 && NVT % NA == 0, "whole runs of column tiles per wave");
        using V4 = typename std::conditional<sizeof(T) == 2, bf16x4, f32x4>::type;
        const int rt = (w * NA) / NVT, ct0 = w * NA - rt * NVT;
        const float gC = sGam[CH - 1];
        if (vs == 0) {  // the same for every slab (K is staged by then)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            // (row d of K^T, token t) = K[t][d], scaled by exp(G_C - G_t)
            adv_a[kb] = frag_oct(sK, LK, 16 * rt, 32 * kb, l);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              adv_a[kb][e] = from_f<T>(to_f(adv_a[kb][e]) * sDte[32 * kb + 8 * (l >> 4) + e]);
          }
        }
#pragma unroll
        for (int m = 0; m < NA; ++m) {
          const int ct = ct0 + m, d0 = 16 * rt + 4 * (l >> 4), vc = 16 * ct + (l & 15);
          float s0[4];
          run4(sS0t, LK, vc, d0, s0);
          f32x4 acc = {gC * s0[0], gC * s0[1], gC * s0[2], gC * s0[3]};
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) mma(acc, adv_a[kb], frag_kc(sRt, LC, 16 * ct, 32 * kb, l));
          *reinterpret_cast<V4*>(sS1t + (vs + vc) * LK + d0) =
              V4{from_f<T>(acc[0]), from_f<T>(acc[1]), from_f<T>(acc[2]), from_f<T>(acc[3])};
        }
      }
    }
    __syncthreads();
  }
  // block reduce <dS_C, S0>
  {
    const float x = wave_sum64(sdot);
    if (l == 0) sRed[w] = x;
  }

  // ---- K phase --------------------------------------------------------------------------------------------
  // The next chunk's reads are issued unconditionally (the last chunk of a workgroup reads its own chunk again,
  // 0.3% of the traffic): after a conditional block the compiler could not count the loads in flight and would
  // wait for all of them at the first reuse of a register of the chunk's earlier reads.
  T* sdq = slab;             // CH x LK   dq staging
  T* sdk = sdq + CH * LK;    // CH x LK   dk staging
  T* sD = sdk + CH * LK;     // CH x LC   D = dA o beta_i E,  column-major (element (r, c) at c * LC + r)
  T* sdPm = sD + CH * LC;    // CH x LC   dP o s E,         column-major

  const int lg = l >> 4;  // lane group: rows 4*lg .. 4*lg+3 of each tile
  float gam[4], dte[4], bet[4], Grow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * rb + acc_row(i, l);
    Grow[i] = sG[r];
    gam[i] = sGam[r];
    dte[i] = sDte[r];
    bet[i] = sB[r];
  }
  // row dots from the V-phase accumulators (this half's columns); dX = -dY S0^T, so rx = dX . k = -aKY . k
  float rq[4] = {0.f, 0.f, 0.f, 0.f}, rk[4] = {0.f, 0.f, 0.f, 0.f}, rx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < HK; ++j) {
    float qv[4], uv[4], kv[4];
    acc_vals(sQ, LK, 16 * rb, 16 * (HK * hf + j), qv, l);
    acc_vals(sU, LK, 16 * rb, 16 * (HK * hf + j), uv, l);
    if constexpr (SEPU) acc_vals(sK, LK, 16 * rb, 16 * (HK * hf + j), kv, l);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      rq[i] += aQg[j][i] * qv[i];
      rk[i] += aKd[j][i] * uv[i];
      rx[i] -= aKY[j][i] * (SEPU ? kv[i] : uv[i]);
    }
  }
  load_first(cnext, false, false);

  // dA = -dY R^T, strict lower; with KK and QK recomputed: D, dPm, dbeta_A and the dG row/col sums
  float rz[4] = {0.f, 0.f, 0.f, 0.f}, dbA[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < HC; ++j) {
    const int n = HC * hf + j;
    f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
    mma_blk<true, true, K>(kk, sK, LK, 16 * rb, sU, LK, 16 * n, l);
    mma_blk<true, true, K>(qk, sQ, LK, 16 * rb, sU, LK, 16 * n, l);
    f32x4 z, Dt, Wt;
    const int cc = 16 * n + acc_col(l);
    const float Gc = sG[cc];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * rb + acc_row(i, l);
      // e = exp(G_r - G_c) on and below the diagonal, computed unconditionally (min(., 0) keeps it finite) and
      // masked by a select: no branch around the exp (written as `cond ? exp : 0` it compiled into an exec-mask
      // branch per element, each waiting for every LDS read in flight).  With u = dA e (strictly below) and
      // w = dP s e:  D = u beta_r,  dPm = w,  dbeta_A += u (K U^T),  z = dP P + dA A = w (Q U^T) + D (K U^T)
      const float ev = __expf(fminf(Grow[i] - Gc, 0.f));
      const float e = r >= cc ? ev : 0.f;
      const float uu = r > cc ? -aDA[j][i] * e : 0.f;
      const float wv = aP[j][i] * (scale * e);
      const float Dv = uu * bet[i];
      Dt[i] = Dv;
      Wt[i] = wv;
      dbA[i] += uu * kk[i];
      z[i] = wv * qk[i] + Dv * kk[i];
      rz[i] += z[i];
    }
    // the lane's four rows of column cc are contiguous in the column-major tiles: one vector store each
    {
      using V4 = typename std::conditional<sizeof(T) == 2, bf16x4, f32x4>::type;
      const int r0 = 16 * rb + acc_row(0, l);
      *reinterpret_cast<V4*>(sD + cc * LC + r0) = V4{from_f<T>(Dt[0]), from_f<T>(Dt[1]), from_f<T>(Dt[2]),
                                                     from_f<T>(Dt[3])};
      *reinterpret_cast<V4*>(sdPm + cc * LC + r0) = V4{from_f<T>(Wt[0]), from_f<T>(Wt[1]), from_f<T>(Wt[2]),
                                                       from_f<T>(Wt[3])};
    }
    const float cs = colsum_tile(z);
    if (lg == 0) sColZ[rb][cc] = cs;
  }
  // Per-row sums over this half's columns: the 24 partials of a lane (6 quantities x its 4 rows, value index
  // 4 q + i) are summed over the 16 lanes of the lane group by a reduce-scatter -- each DPP exchange halves the
  // number of values held (12 pairs with the mirrored lane, 6 with the half-row mirror, 3 with lane ^ 2, then
  // lane ^ 1) -- instead of a 4-step butterfly per value.  Lane p (in its group) ends with the total of value
  // f0 = (p & 1) + s and, like lane p ^ 1, of value f1 = 2 + s (s = 3 bit1 + 6 bit2 + 12 bit3 of p), and writes
  // them to sRow for this half.
  {
    float a[24];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = rq[i];
      a[4 + i] = rk[i];
      a[8 + i] = dbV[i];
      a[12 + i] = rx[i];
      a[16 + i] = dbA[i];
      a[20 + i] = rz[i];
    }
    const int p = l & 15;
    rs_round<12, 0x140>(a, (p >> 3) & 1);  // row_mirror: lane 15 - p
    rs_round<6, 0x141>(a, (p >> 2) & 1);   // row_half_mirror: lane 7 - p within the half-row
    rs_round<3, 0x4e>(a, (p >> 1) & 1);    // quad_perm [2,3,0,1]: lane p ^ 2
    rs_round<1, 0xb1>(a, p & 1);           // quad_perm [1,0,3,2]: lane p ^ 1
    const float z1 = dpp_sum_step<0xb1>(a[2]);
    const int sb = 3 * ((p >> 1) & 1) + 6 * ((p >> 2) & 1) + 12 * ((p >> 3) & 1);
    const int f0 = sb + (p & 1), f1 = sb + 2;
    sRow[hf][f0 >> 2][16 * rb + 4 * lg + (f0 & 3)] = a[0];
    if ((p & 1) == 0) sRow[hf][f1 >> 2][16 * rb + 4 * lg + (f1 & 3)] = z1;
  }
  __syncthreads();
  load_b(cnext, 0, !is_odd(cnext));
  // dq = s gamma dQg + dPm U.  (Here and below every tile of a product is computed before any is stored: with no
  // LDS store in between, the row block's A fragments are read once for all column tiles.)
  {
    f32x4 t[HK];
#pragma unroll
    for (int j = 0; j < HK; ++j) {
      t[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma_blk<false, false, CH>(t[j], sdPm, LC, 16 * rb, sU, LK, 16 * (HK * hf + j), l);
    }
#pragma unroll
    for (int j = 0; j < HK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rb + acc_row(i, l), d = 16 * (HK * hf + j) + acc_col(l);
        sdq[r * LK + d] = from_f<T>(scale * gam[i] * aQg[j][i] + t[j][i]);
      }
  }
  if constexpr (!SEPU) {
    // dk = dte dKd + dPm^T Q + D K + D^T K - beta gamma dKY
    f32x4 t[HK];
#pragma unroll
    for (int j = 0; j < HK; ++j) {
      const int n = HK * hf + j;
      t[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma_blk<true, false, CH>(t[j], sdPm, LC, 16 * rb, sQ, LK, 16 * n, l);
      mma_blk<false, false, CH>(t[j], sD, LC, 16 * rb, sK, LK, 16 * n, l);
      mma_blk<true, false, CH>(t[j], sD, LC, 16 * rb, sK, LK, 16 * n, l);
    }
#pragma unroll
    for (int j = 0; j < HK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rb + acc_row(i, l), d = 16 * (HK * hf + j) + acc_col(l);
        sdk[r * LK + d] = from_f<T>(dte[i] * aKd[j][i] + t[j][i] - bet[i] * gam[i] * aKY[j][i]);
      }
  } else {
    // read side: dk = D U - beta gamma dKY;  write side (kept in aKd until its staging area is free):
    // du = dte dKd + dPm^T Q + D^T K
    f32x4 t[HK];
#pragma unroll
    for (int j = 0; j < HK; ++j) {
      const int n = HK * hf + j;
      f32x4 t2 = {0.f, 0.f, 0.f, 0.f};
      t[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      mma_blk<false, false, CH>(t[j], sD, LC, 16 * rb, sU, LK, 16 * n, l);
      mma_blk<true, false, CH>(t2, sdPm, LC, 16 * rb, sQ, LK, 16 * n, l);
      mma_blk<true, false, CH>(t2, sD, LC, 16 * rb, sK, LK, 16 * n, l);
#pragma unroll
      for (int i = 0; i < 4; ++i) aKd[j][i] = dte[i] * aKd[j][i] + t2[i];
    }
#pragma unroll
    for (int j = 0; j < HK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * rb + acc_row(i, l), d = 16 * (HK * hf + j) + acc_col(l);
        sdk[r * LK + d] = from_f<T>(t[j][i] - bet[i] * gam[i] * aKY[j][i]);
      }
  }
  // dbeta and the per-row part of dG (first half, one lane per row)
  if (hf == 0 && (l & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * rb + acc_row(i, l);
      const float q_ = sRow[0][0][r] + sRow[1][0][r], k_ = sRow[0][1][r] + sRow[1][1][r];
      const float v_ = sRow[0][2][r] + sRow[1][2][r], x_ = sRow[0][3][r] + sRow[1][3][r];
      const float a_ = sRow[0][4][r] + sRow[1][4][r], z_ = sRow[0][5][r] + sRow[1][5][r];
      const float db = gam[i] * x_ + v_ + a_;
      if (dbeta && r < nvalid) dbeta[row0 + (int64_t)r * H] = db;
      sdG[r] = scale * gam[i] * q_ - dte[i] * k_ + bet[i] * gam[i] * x_ + z_;
      sLast[r] = dte[i] * k_;
    }
  }
  __syncthreads();
  s2g_rows<T, CH, K, ITH, INTRA_NT>(dq + row0 * K, (int64_t)H * K, sdq, LK, nvalid, tid);
  s2g_rows<T, CH, K, ITH, INTRA_NT>(dk + row0 * K, (int64_t)H * K, sdk, LK, nvalid, tid);
  if constexpr (SEPU) {
    // du staged in the D and dPm regions, free once every wave has passed the barrier above
    T* sdu = sD;
#pragma unroll
    for (int j = 0; j < HK; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sdu[(16 * rb + acc_row(i, l)) * LK + 16 * (HK * hf + j) + acc_col(l)] = from_f<T>(aKd[j][i]);
    __syncthreads();
    s2g_rows<T, CH, K, ITH, INTRA_NT>(du + row0 * K, (int64_t)H * K, sdu, LK, nvalid, tid);
  }
  // The next chunk overwrites the staged rows read above.  Wave 0's reverse cumsum below reads only sdG, sColZ,
  // sLast and sRed, which the next chunk writes after barriers that wave 0 must reach first, so the other waves
  // go on into the next chunk meanwhile.
  __syncthreads();
  if (w == 0) {
    // dG_r -= colsum_r;  dG_last += sum_r dte_r rk_r + gamma_C <dS_C, S0>;  dg = reverse cumsum of dG
    float x = sdG[l] - (sColZ[0][l] + sColZ[1][l] + sColZ[2][l] + sColZ[3][l]);
    float last = wave_sum64(sLast[l]);
    float red = 0.f;
#pragma unroll
    for (int i = 0; i < IW; ++i) red += sRed[i];
    last += sGam[CH - 1] * red;
    if (l == CH - 1) x += last;
    const float incl = wave_inclusive_scan(x);
    const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), 63));
    if (l < nvalid) dg[row0 + (int64_t)l * H] = total - incl + x;
  }
  it = it_next;
  ci = cnext;
  }
}

// ---------------------------------------------------------------------------------------------------------
template <typename T, int K, bool SEPU, int BV>
static hipError_t bwd_state_bv(const ChunkArgs& a, bool local) {
  dim3 grid(a.V / BV * a.B * a.H);
  auto go = [&](auto kern) {
    kern<<<grid, state_threads<BV>(), 0, a.stream>>>(
        static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.u),
        static_cast<const T*>(a.dout), a.beta, static_cast<const T*>(a.ws.Tm), static_cast<const T*>(a.ws.P),
        a.ws.Gc, a.dhT, a.dh0, static_cast<T*>(a.ws.dhs), static_cast<T*>(a.ws.dYs), a.T, a.H, a.V, a.NT,
        a.scale, a.ns);
    return hipGetLastError();
  };
  return local ? go(bwd_state_kernel<T, K, BV, SEPU, false>) : go(bwd_state_kernel<T, K, BV, SEPU, true>);
}

template <typename T, int K, bool SEPU>
static hipError_t bwd_state_k(const ChunkArgs& a, bool local) {
  if constexpr (sizeof(T) == 2 && !SEPU) {
    if (narrow_sweep_blocks(a, a.V / 32)) return bwd_state_bv<T, K, SEPU, 32>(a, local);
  }
  return bwd_state_bv<T, K, SEPU, 64>(a, local);
}

template <typename T, int K, int V, bool SEPU, bool HALF>
static hipError_t bwd_intra_launch(const ChunkArgs& a) {
  constexpr int VS = sizeof(T) == 2 ? 64 : 32;
  // persistent: one workgroup per CU (the LDS use allows no more), each looping over chunks (HALF: chunk pairs)
  const int nitem = (HALF ? (a.NT + 1) / 2 : a.NT) * a.B * a.H;
  dim3 grid(std::min(nitem, device_cu_count()));
  bwd_intra_kernel<T, K, V, VS, SEPU, HALF><<<grid, ITH, 0, a.stream>>>(
      static_cast<const T*>(a.q), static_cast<const T*>(a.k), static_cast<const T*>(a.u),
      static_cast<const T*>(a.v), a.beta, static_cast<const T*>(a.dout),
      a.ws.Gc, static_cast<const T*>(a.ws.hs), static_cast<const T*>(a.ws.Rs), static_cast<const T*>(a.ws.dhs),
      static_cast<const T*>(a.ws.dYs), static_cast<T*>(a.dq), static_cast<T*>(a.dk), static_cast<T*>(a.du),
      static_cast<T*>(a.dv), a.dg, a.dbeta, a.T, a.H, a.NT, a.B * a.H, a.scale);
  return hipGetLastError();
}

template <typename T, int K, int V, bool SEPU>
static hipError_t bwd_intra_kv(const ChunkArgs& a) {
  if constexpr (sizeof(T) == 2 && !SEPU && V <= 128) {
    if (a.hstride == 2) return bwd_intra_launch<T, K, V, SEPU, true>(a);
  }
  if (a.hstride != 1) return hipErrorInvalidValue;  // the stash layout this build's forward would not write
  return bwd_intra_launch<T, K, V, SEPU, false>(a);
}

template <typename T, int K, bool SEPU>
static hipError_t bwd_intra_k(const ChunkArgs& a) {
  if (a.V == 64) return bwd_intra_kv<T, K, 64, SEPU>(a);
  if (a.V == 128) return bwd_intra_kv<T, K, 128, SEPU>(a);
  if (a.V == 256) return bwd_intra_kv<T, K, 256, SEPU>(a);
  return hipErrorInvalidValue;
}

template <bool SEPU>
static hipError_t bwd_state_dispatch(const ChunkArgs& a, bool local) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return bwd_state_k<bf16, 64, SEPU>(a, local);
    if (a.K == 128) return bwd_state_k<bf16, 128, SEPU>(a, local);
  } else if constexpr (!SEPU) {  // separate write keys: bf16 only
    if (a.K == 64) return bwd_state_k<float, 64, SEPU>(a, local);
  }
  return hipErrorInvalidValue;
}

template <bool SEPU>
static hipError_t bwd_intra_dispatch(const ChunkArgs& a) {
  if (a.dtype == DT_BF16) {
    if (a.K == 64) return bwd_intra_k<bf16, 64, SEPU>(a);
    if (a.K == 128) return bwd_intra_k<bf16, 128, SEPU>(a);
  } else if constexpr (!SEPU) {  // separate write keys: bf16 only
    if (a.K == 64) return bwd_intra_k<float, 64, SEPU>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_state(const ChunkArgs& a, bool local) {
  return a.u ? bwd_state_dispatch<true>(a, local) : bwd_state_dispatch<false>(a, local);
}

hipError_t launch_bwd_intra(const ChunkArgs& a) {
  return a.u ? bwd_intra_dispatch<true>(a) : bwd_intra_dispatch<false>(a);
}

}  // namespace gdn
