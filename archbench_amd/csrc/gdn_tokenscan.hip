// Exact fp32 token scan of the n-step gated DeltaNet, forward and reverse-time backward: the reference's
// "triton" / "ref" scan (archbench/layers/nsgdn.py:80-154, ops :162-216; the recurrence of nsgdn_ref, :408-417).
// Per token t of a (b, h) sequence, with the state S [V, K] fp32 from zero (or from an initial state):
//     S <- e^{la_t} S;   r_t = v_t - S k_t;   S <- S + r_t u_t^T;   y_t = S q_t.
// Rows of S are independent given the token stream.  A workgroup of eight waves owns 64 rows; eight lanes share a
// row, lane part l & 7 holding K / 8 of its entries in registers, so a row's dot products (S k, S q, G u) are a
// partial sum per lane and three DPP steps inside the 8-lane group.  k, u, q of a token are workgroup-uniform and
// reach the lanes through LDS, staged a block of tokens at a time (double-buffered: the next block is staged while
// one computes, one barrier per block).  Every CT tokens the forward stores S (the checkpoint the backward restarts
// from) in [K][V] order.
// The backward walks the checkpoints in reverse and each chunk in groups of four tokens, last first: it recomputes
// a group's states forward from the state entering the group (stored by a forward pass over the chunk from its
// checkpoint), keeping e^{la} S before each token's update in registers and accumulating dq = sum_rows S_t^T dy_t,
// then runs the group's tokens backward with the state gradient G [V, K] in registers beside S:
//     G += dy_t q_t^T;  dv_t = G u_t;  du_t = sum_rows G r_t;  G -= dv_t k_t^T;
//     dk_t = -sum_rows (e^{la} S_{t-1}) dv_t;  dla_t = sum (G o e^{la} S_{t-1});  G <- e^{la_t} G.
// Sums over rows are a reduce-scatter over the wave's 8 rows (lane swaps and DPP, no LDS crossbar), then over the
// eight waves through LDS (a fixed order, no atomics), then over a head's V / 64 workgroups through partial rows that
// the host adds.
#include <hip/hip_runtime.h>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int TS_CT = 32;                    // tokens between checkpoints
constexpr int TS_GS = 4;                     // tokens per group of the backward (decayed states held in registers)
constexpr int TS_ROWS = 64;                  // state rows per workgroup
constexpr int TS_LB = 3;                     // log2 of the lanes per row (16 lanes: slower, spills)
constexpr int TS_LPR = 1 << TS_LB;           // lanes per row
constexpr int TS_THREADS = TS_LPR * TS_ROWS;
constexpr int TS_WAVES = TS_THREADS / 64;    // each wave holds 64 / TS_LPR rows

// The block / group barrier orders LDS only (the staged vectors and the row sums): __syncthreads() would also wait
// for every global load in flight, the next block's included, and so expose a memory latency per barrier.
__device__ __forceinline__ void ts_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// A zero the compiler cannot see through, added to a workgroup-uniform index so that the load is a vector load: a
// scalar load would be waited for at the next barrier (scalar loads and LDS share one wait counter).
__device__ __forceinline__ int ts_vector_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// sum over the lanes of a row, left in each of them: quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror (lane
// p <- 7 - p) adds the other quad of an 8-lane group and row_mirror (p <- 15 - p) the other half of a 16-lane row
__device__ __forceinline__ float ts_row_sum(float x) {
  x = dpp_sum_step<0x4e>(dpp_sum_step<0xb1>(x));
  if constexpr (TS_LB >= 3) x = dpp_sum_step<0x141>(x);
  if constexpr (TS_LB >= 4) x = dpp_sum_step<0x140>(x);
  return x;
}

// Reduce-scatter over a wave's 64 / TS_LPR rows: N values per lane (its part's local columns), summed over the lanes
// that share l & (TS_LPR - 1) (lane bits TS_LB .. 5).  With R = N TS_LPR / 64, lane l ends with the sums of local
// columns m + R (l >> TS_LB), m < R, in a[0 .. R).  Each round pairs lanes that differ in one bit and hold the same column set: one keeps the lower
// half of its set, the other the upper half, and each adds what its partner sends.
template <int N>
__device__ __forceinline__ void ts_rows_rs(float (&a)[N], int l) {
  // bit 5: v_permlane32_swap of (a[m], a[m + N/2]) gives the lower half-wave its partner's a[m] and the upper half
  // its partner's a[m + N/2] (each keeps its own in the other result), so one add finishes the round
#pragma unroll
  for (int m = 0; m < N / 2; ++m) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[m]), __float_as_uint(a[m + N / 2]), false, false);
    a[m] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  if constexpr (TS_LB > 4) return;
  // bit 4: the same with v_permlane16_swap between even and odd 16-lane rows
#pragma unroll
  for (int m = 0; m < N / 4; ++m) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[m]), __float_as_uint(a[m + N / 4]), false, false);
    a[m] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  if constexpr (TS_LB > 3) return;
  // bit 3: row_ror:8 pairs lanes p and p ^ 8 of a 16-lane row
  const int b3 = (l >> 3) & 1;
#pragma unroll
  for (int m = 0; m < N / 8; ++m) {
    const float keep = b3 ? a[m + N / 8] : a[m], send = b3 ? a[m] : a[m + N / 8];
    a[m] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0x128, 0xf, 0xf, true));
  }
}

// A token's k, u, q in LDS: per vector eight blocks of K / 8 floats, each padded by 4 so that the eight lanes of a
// row (one per block) read different banks with 16-byte reads.  Piece p < 3 K / 4 of a token (or one of the K / 4
// pieces of u alone) is one float4, loaded into a register well ahead of its token and stored here before it.
template <int K>
struct TokStage {
  static constexpr int KQ = K / TS_LPR, K4 = K / 4, LD = KQ + 4, VEC = TS_LPR * LD, SIZE = 3 * VEC;
  static __device__ __forceinline__ void load(const float* kp, const float* up, const float* qp, int64_t t, int tid,
                                              bool kq, f32x4& x) {  // tid: the piece
    const int vec = tid / K4, e4 = tid - vec * K4;
    if (kq ? tid < 3 * K4 : vec == 1) {
      const float* src = vec == 0 ? kp : vec == 1 ? up : qp;
      x = *reinterpret_cast<const f32x4*>(src + t * K + 4 * e4);
    }
  }
  static __device__ __forceinline__ void stage(float* sv, int tid, bool kq, const f32x4& x) {
    const int vec = tid / K4, c = 4 * (tid - vec * K4), qd = c / KQ;
    if (kq ? tid < 3 * K4 : vec == 1) *reinterpret_cast<f32x4*>(sv + vec * VEC + qd * LD + c - qd * KQ) = x;
  }
};

// this lane's quarter of a staged vector, as KQ floats through 16-byte LDS reads
template <int KQ>
__device__ __forceinline__ void ts_read(const float* p, float (&o)[KQ]) {
#pragma unroll
  for (int m = 0; m < KQ / 4; ++m) {
    const f32x4 t = reinterpret_cast<const f32x4*>(p)[m];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[4 * m + e] = t[e];
  }
}

// Tokens per block of the forward: a block's k, u, q are staged through LDS together (loaded a block ahead), so the
// workgroup meets at one barrier per block and its waves run through the block's tokens unsynchronised.
constexpr int TS_TB = 8;
static_assert(TS_CT % TS_TB == 0, "checkpoints fall on block starts");

// grid B * H * NB (NB = ceil(V / 64)) workgroups of TS_THREADS (512) threads: workgroup x -> (b h, row block vb)
template <int K>
__global__ __launch_bounds__(TS_THREADS) void token_scan_fwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ u, const float* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ h0, float* __restrict__ y, float* __restrict__ r,
    float* __restrict__ st, float* __restrict__ hT, int T_, int H, int V, int NCH, int NB) {
  using TS = TokStage<K>;
  constexpr int KQ = TS::KQ, PER = 3 * TS::K4, NL = (TS_TB * PER + TS_THREADS - 1) / TS_THREADS;
  __shared__ __attribute__((aligned(16))) float sv[2][TS_TB][TS::SIZE];
  const int tid = threadIdx.x, l = lane_id(), qd = l & (TS_LPR - 1);
  const int pid = blockIdx.x, bh = pid / NB, vb = pid - bh * NB;
  const int b = bh / H, h = bh - b * H;
  const int vi = vb * TS_ROWS + (tid >> TS_LB);
  const bool on = vi < V;
  const int vc = on ? vi : V - 1;  // rows past V compute on row V-1 and store nothing
  // states [B, H, K, V] (fla's layout): entry (row vi, column qd KQ + j) at cb + j V
  const int64_t cb = (int64_t)bh * K * V + (int64_t)qd * KQ * V + vi;
  float S[KQ];
#pragma unroll
  for (int j = 0; j < KQ; ++j) S[j] = h0 && on ? h0[cb + (int64_t)j * V] : 0.f;
  float* stb = st + (int64_t)bh * NCH * K * V + (int64_t)qd * KQ * V + vi;
  const int64_t tok_first = (int64_t)b * T_ * H + h;
  // block t0's vectors: thread piece e < TS_TB * PER is float4 e % PER (k, u, q in order) of token t0 + e / PER
  f32x4 xr[NL];
  float vn[TS_TB], ln[TS_TB];  // the next block's v (this row) and la, loaded a block ahead
  const int zv = ts_vector_zero();
  auto load_block = [&](int t0) {
#pragma unroll
    for (int m = 0; m < NL; ++m) {
      const int e = tid + m * TS_THREADS, i = e / PER, rem = e - i * PER;
      if (e < TS_TB * PER && t0 + i < T_) TS::load(k, u, q, tok_first + (int64_t)(t0 + i) * H, rem, true, xr[m]);
    }
#pragma unroll
    for (int i = 0; i < TS_TB; ++i) {
      const int64_t tk = tok_first + (int64_t)min(t0 + i, T_ - 1) * H;
      vn[i] = v[tk * V + vc];
      ln[i] = la[tk + zv];
    }
  };
  auto stage_block = [&](float (*dst)[TS::SIZE]) {
#pragma unroll
    for (int m = 0; m < NL; ++m) {
      const int e = tid + m * TS_THREADS, i = e / PER, rem = e - i * PER;
      if (e < TS_TB * PER) TS::stage(dst[i], rem, true, xr[m]);
    }
  };
  float vcur[TS_TB], lcur[TS_TB];
  load_block(0);  // T_ >= 1 here (the host returns before launching an empty scan)
  stage_block(sv[0]);
#pragma unroll
  for (int i = 0; i < TS_TB; ++i) vcur[i] = vn[i], lcur[i] = ln[i];
  if (TS_TB < T_) load_block(TS_TB);
  ts_barrier();
  for (int t0 = 0, blk = 0; t0 < T_; t0 += TS_TB, ++blk) {
    if (t0 % TS_CT == 0 && on) {
      const int64_t c = t0 / TS_CT;
#pragma unroll
      for (int j = 0; j < KQ; ++j) stb[(c * K + j) * V] = S[j];
    }
#pragma unroll
    for (int i = 0; i < TS_TB; ++i) {
      if (t0 + i >= T_) break;
      const int64_t tok = tok_first + (int64_t)(t0 + i) * H;
      const float a = expf(lcur[i]);
      const float* sk = sv[blk & 1][i] + qd * TS::LD;
      float kk[KQ];
      ts_read<KQ>(sk, kk);
      float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KQ; ++j) {
        S[j] *= a;
        d[j & 3] = fmaf(S[j], kk[j], d[j & 3]);
      }
      const float rr = vcur[i] - ts_row_sum((d[0] + d[1]) + (d[2] + d[3]));
      float uu[KQ], qq[KQ];
      ts_read<KQ>(sk + TS::VEC, uu);
      ts_read<KQ>(sk + 2 * TS::VEC, qq);
      float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KQ; ++j) {
        S[j] = fmaf(rr, uu[j], S[j]);
        e[j & 3] = fmaf(S[j], qq[j], e[j & 3]);
      }
      const float yy = ts_row_sum((e[0] + e[1]) + (e[2] + e[3]));
      if (on && qd == 0) r[tok * V + vi] = rr;
      if (on && qd == 1) y[tok * V + vi] = yy;
    }
    if (t0 + TS_TB < T_) {  // stage the next block (loaded a block ago), load the one after it
      stage_block(sv[(blk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TS_TB; ++i) vcur[i] = vn[i], lcur[i] = ln[i];
      if (t0 + 2 * TS_TB < T_) load_block(t0 + 2 * TS_TB);
    }
    ts_barrier();  // the block's vectors read by every lane; the next block's staged
  }
  if (hT && on) {
#pragma unroll
    for (int j = 0; j < KQ; ++j) hT[cb + (int64_t)j * V] = S[j];
  }
}

// The row sums of a group's steps: each wave's column sums (after ts_rows_rs) and its dla go to LDS slots of their
// own (vector, token), and after the group's barrier the eight waves are added in a fixed order and stored as the
// workgroup's partial rows (double-buffered by group parity).
template <int K>
struct TokSums {
  float col[2][3][TS_GS][TS_WAVES][K];  // [parity][dq, du, dk][token][wave][column]
  float sca[2][TS_GS][TS_WAVES];        // [parity][token][wave]: dla
  // this wave's reduce-scattered sums of local columns (part l & (TS_LPR - 1)) into slot (vec, i)
  template <int KQ>
  __device__ __forceinline__ void put(int par, int vec, int i, const float (&a)[KQ], int l) {
    constexpr int R = KQ * TS_LPR / 64;
    const int w = wave_id(), c0 = (l & (TS_LPR - 1)) * KQ + R * (l >> TS_LB);
#pragma unroll
    for (int m = 0; m < R; ++m) col[par][vec][i][w][c0 + m] = a[m];
  }
  // the waves' values added as a pairwise tree (a fixed order)
  template <typename F>
  static __device__ __forceinline__ float tree(F&& x) {
    float a[TS_WAVES];
#pragma unroll
    for (int w = 0; w < TS_WAVES; ++w) a[w] = x(w);
#pragma unroll
    for (int h = TS_WAVES / 2; h >= 1; h /= 2) {
#pragma unroll
      for (int w = 0; w < h; ++w) a[w] = a[2 * w] + a[2 * w + 1];
    }
    return a[0];
  }
  __device__ __forceinline__ float col_sum(int par, int vec, int i, int c) const {
    return tree([&](int w) { return col[par][vec][i][w][c]; });
  }
  __device__ __forceinline__ float sca_sum(int par, int i) const {
    return tree([&](int w) { return sca[par][i][w]; });
  }
};
static_assert(TS_LB >= 3 && TS_LB <= 4, "row sums and reduce-scatter rounds cover 8 or 16 lanes per row");

// Partials: gqp, gup, gkp [NB][B*T*H][K], glap [NB][B*T*H]; sc [B*H*NB][TS_CT / TS_GS][K / TS_LPR][TS_THREADS] scratch of
// the chunk's group-start states.
// Per chunk (last first), in groups of TS_GS tokens: a forward pass from the checkpoint stores the state entering each
// group but the first and last (the last stays in registers); then, group by group from the last, the group's tokens
// are recomputed forward from its start state with each decayed state e^{la} S_{t-1} kept in registers (and dq
// accumulated), and walked backward.  A short last group is padded with identity tokens (la = 0, zero vectors and
// row values), which change neither S nor G, and whose sums are not stored.  Both passes stage a group's vectors
// through LDS (and load its row values) a group ahead: one barrier per group.
template <int K>
__global__ __launch_bounds__(TS_THREADS) void token_scan_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ u, const float* __restrict__ la,
    const float* __restrict__ r, const float* __restrict__ st, const float* __restrict__ gy,
    const float* __restrict__ dhT, float* __restrict__ gv, float* __restrict__ gqp, float* __restrict__ gup,
    float* __restrict__ gkp, float* __restrict__ glap, float* __restrict__ dh0, float* __restrict__ sc, int T_, int H,
    int V, int NCH, int NB, int64_t ntok) {
  using TS = TokStage<K>;
  constexpr int KQ = TS::KQ, NGS = TS_CT / TS_GS, PER = 3 * TS::K4;
  static_assert(TS_GS * PER <= TS_THREADS, "one piece of a group's vectors per thread");
  __shared__ __attribute__((aligned(16))) float sv[2][TS_GS][TS::SIZE];
  __shared__ TokSums<K> sums;
  const int tid = threadIdx.x, l = lane_id(), qd = l & (TS_LPR - 1);
  const int pid = blockIdx.x, bh = pid / NB, vb = pid - bh * NB;
  const int b = bh / H, h = bh - b * H;
  const int vi = vb * TS_ROWS + (tid >> TS_LB);
  const bool on = vi < V;
  const float* stb = st + (int64_t)bh * NCH * K * V + (int64_t)qd * KQ * V + vi;
  float* scw = sc + (int64_t)pid * NGS * KQ * TS_THREADS + tid;
  float* const gout[3] = {gqp + (int64_t)vb * ntok * K, gup + (int64_t)vb * ntok * K, gkp + (int64_t)vb * ntok * K};
  float* gl_b = glap + (int64_t)vb * ntok;
  const int zv = ts_vector_zero();
  const int pi = tid / PER, prem = tid - pi * PER;  // this thread's piece of a group's vectors: token pi, piece prem
  f32x4 xr;                                         // ... of the next group, loaded a group ahead
  float nla[TS_GS], nr[TS_GS], ngy[TS_GS];          // the next group's row values
  float cla[TS_GS], cr[TS_GS], cgy[TS_GS];          // the current group's
  // a group's tokens tok_at(i), i < TS_GS (tok < 0: an identity token); kq: k, q and dy too (else u and r alone)
  auto load_grp = [&](auto&& tok_at, bool kq) {
    if (pi < TS_GS) {
      const int64_t tk = tok_at(pi);
      if (tk >= 0) TS::load(k, u, q, tk, prem, kq, xr);
      else xr = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < TS_GS; ++i) {
      const int64_t tk = tok_at(i);
      nla[i] = tk >= 0 ? la[tk + zv] : 0.f;
      nr[i] = tk >= 0 && on ? r[tk * V + vi] : 0.f;
      ngy[i] = tk >= 0 && on && kq ? gy[tk * V + vi] : 0.f;
    }
  };
  auto stage_grp = [&](int buf, bool kq) {
    if (pi < TS_GS) TS::stage(sv[buf][pi], prem, kq, xr);
#pragma unroll
    for (int i = 0; i < TS_GS; ++i) cla[i] = nla[i], cr[i] = nr[i], cgy[i] = ngy[i];
  };
  int par = 0;  // parity of the group: sv[par & 1] holds its vectors, sums[par & 1] takes its row sums
  const int64_t cb = (int64_t)bh * K * V + (int64_t)qd * KQ * V + vi;  // [B, H, K, V] states, as in the forward
  float G[KQ], S[KQ];
#pragma unroll
  for (int j = 0; j < KQ; ++j) G[j] = dhT && on ? dhT[cb + (int64_t)j * V] : 0.f;
  for (int c = NCH - 1; c >= 0; --c) {
    const int n = min(TS_CT, T_ - c * TS_CT), ng = (n + TS_GS - 1) / TS_GS;
    const int64_t tok0 = ((int64_t)b * T_ + (int64_t)c * TS_CT) * H + h;
    auto tok_in = [&](int g, int i) -> int64_t {
      const int t = g * TS_GS + i;
      return t < n ? tok0 + (int64_t)t * H : -1;
    };
#pragma unroll
    for (int j = 0; j < KQ; ++j) S[j] = on ? stb[((int64_t)c * K + j) * V] : 0.f;
    // forward from the checkpoint to the last group's start, storing the start states of groups 1 .. ng - 2
    if (ng > 1) {
      load_grp([&](int i) { return tok_in(0, i); }, false);
      stage_grp(par & 1, false);
      if (ng > 2) load_grp([&](int i) { return tok_in(1, i); }, false);
      ts_barrier();
      for (int g = 0; g < ng - 1; ++g, ++par) {
        const int p = par & 1;
        if (g > 0) {
#pragma unroll
          for (int j = 0; j < KQ; ++j) scw[((int64_t)g * KQ + j) * TS_THREADS] = S[j];
        }
#pragma unroll
        for (int i = 0; i < TS_GS; ++i) {
          float uu[KQ];
          ts_read<KQ>(sv[p][i] + TS::VEC + qd * TS::LD, uu);
          const float a = expf(cla[i]);
#pragma unroll
          for (int j = 0; j < KQ; ++j) S[j] = fmaf(cr[i], uu[j], S[j] * a);
        }
        if (g + 1 < ng - 1) {
          stage_grp((par + 1) & 1, false);
          if (g + 2 < ng - 1) load_grp([&](int i) { return tok_in(g + 2, i); }, false);
        }
        ts_barrier();
      }
    }
    // groups last to first: TS_GS forward steps (tokens 0 .. TS_GS - 1 of the group), then TS_GS backward steps
    auto flush = [&](int g, int pb) {  // the group's row sums, from LDS slots of parity pb
#pragma unroll
      for (int m = 0; m < (3 * TS_GS * K + TS_THREADS - 1) / TS_THREADS; ++m) {
        const int o = tid + m * TS_THREADS;
        if (o < 3 * TS_GS * K) {
          const int vec = o / (TS_GS * K), rem = o - vec * TS_GS * K, i = rem / K, cc = rem - i * K;
          const int64_t tk = tok_in(g, i);
          if (tk >= 0) gout[vec][tk * K + cc] = sums.col_sum(pb, vec, i, cc);
        }
      }
      if (tid < TS_GS) {
        const int64_t tk = tok_in(g, tid);
        if (tk >= 0) gl_b[tk] = sums.sca_sum(pb, tid);
      }
    };
    load_grp([&](int i) { return tok_in(ng - 1, i); }, true);
    stage_grp(par & 1, true);
    if (ng > 1) load_grp([&](int i) { return tok_in(ng - 2, i); }, true);
    ts_barrier();
    for (int g = ng - 1; g >= 0; --g, ++par) {
      const int p = par & 1;
      if (g < ng - 1) {
        flush(g + 1, p ^ 1);
        if (g == 0) {
#pragma unroll
          for (int j = 0; j < KQ; ++j) S[j] = on ? stb[((int64_t)c * K + j) * V] : 0.f;
        } else {
#pragma unroll
          for (int j = 0; j < KQ; ++j) S[j] = scw[((int64_t)g * KQ + j) * TS_THREADS];
        }
      }
      float Sd[TS_GS][KQ];  // e^{la} S_{t-1} of the group's tokens
#pragma unroll
      for (int s = 0; s < 2 * TS_GS; ++s) {
        const int i = s < TS_GS ? s : 2 * TS_GS - 1 - s;
        const float a = expf(cla[i]), rc = cr[i], gyc = cgy[i];
        const float* sb = sv[p][i] + qd * TS::LD;
        float uu[KQ], t[KQ];
        ts_read<KQ>(sb + TS::VEC, uu);
        if (s < TS_GS) {
#pragma unroll
          for (int j = 0; j < KQ; ++j) {
            S[j] *= a;
            Sd[i][j] = S[j];
            S[j] = fmaf(rc, uu[j], S[j]);
            t[j] = S[j] * gyc;
          }
          ts_rows_rs<KQ>(t, l);
          sums.put(p, 0, i, t, l);
        } else {
          float qq[KQ], kk[KQ];
          ts_read<KQ>(sb + 2 * TS::VEC, qq);
          float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < KQ; ++j) {
            G[j] = fmaf(gyc, qq[j], G[j]);
            d[j & 3] = fmaf(G[j], uu[j], d[j & 3]);
          }
          const float gr = ts_row_sum((d[0] + d[1]) + (d[2] + d[3]));
          const int64_t tok = tok_in(g, i);
          if (on && qd == 0 && tok >= 0) gv[tok * V + vi] = gr;
#pragma unroll
          for (int j = 0; j < KQ; ++j) t[j] = G[j] * rc;
          ts_rows_rs<KQ>(t, l);
          sums.put(p, 1, i, t, l);
          ts_read<KQ>(sb, kk);
#pragma unroll
          for (int j = 0; j < KQ; ++j) {
            G[j] = fmaf(-gr, kk[j], G[j]);
            t[j] = -Sd[i][j] * gr;
          }
          ts_rows_rs<KQ>(t, l);
          sums.put(p, 2, i, t, l);
          float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < KQ; ++j) e[j & 3] = fmaf(G[j], Sd[i][j], e[j & 3]);
          const float gl = wave_sum64((e[0] + e[1]) + (e[2] + e[3]));
          if (l == 0) sums.sca[p][i][wave_id()] = gl;
#pragma unroll
          for (int j = 0; j < KQ; ++j) G[j] *= a;
        }
      }
      if (g > 0) {  // stage the group before (loaded a group ago), load the one before it
        stage_grp((par + 1) & 1, true);
        if (g > 1) load_grp([&](int i) { return tok_in(g - 2, i); }, true);
      }
      ts_barrier();  // the group's vectors read and sums written; the group before staged
    }
    flush(0, (par - 1) & 1);
  }
  // G is now the gradient of the state before the first token: the initial state's
  if (dh0 && on) {
#pragma unroll
    for (int j = 0; j < KQ; ++j) dh0[cb + (int64_t)j * V] = G[j];
  }
}

// ---------------------------------------------------------------------------------------------------------
bool token_scan_supported(int K) { return K == 64 || K == 128; }
int token_scan_ct() { return TS_CT; }
size_t token_scan_scratch_floats(int K) { return (size_t)(TS_CT / TS_GS) * K * TS_ROWS; }

template <int K>
static hipError_t token_scan_k(const TokenScanArgs& a, bool backward) {
  const int NB = (a.V + TS_ROWS - 1) / TS_ROWS, NCH = (a.T + TS_CT - 1) / TS_CT;
  const dim3 grid((unsigned)(a.B * a.H * NB));
  if (!backward) {
    token_scan_fwd_kernel<K><<<grid, TS_THREADS, 0, a.stream>>>(a.q, a.k, a.u, a.v, a.la, a.h0, a.y, a.r, a.st,
                                                                a.hT, a.T, a.H, a.V, NCH, NB);
  } else {
    token_scan_bwd_kernel<K><<<grid, TS_THREADS, 0, a.stream>>>(
        a.q, a.k, a.u, a.la, a.r, a.st, a.dy, a.dhT, a.dv, a.dq_part, a.du_part, a.dk_part, a.dla_part, a.dh0,
        a.scratch, a.T, a.H, a.V, NCH, NB, (int64_t)a.B * a.T * a.H);
  }
  return hipGetLastError();
}

hipError_t launch_token_scan(const TokenScanArgs& a, bool backward) {
  switch (a.K) {
    case 64: return token_scan_k<64>(a, backward);
    case 128: return token_scan_k<128>(a, backward);
  }
  return hipErrorInvalidValue;
}

}  // namespace gdn
