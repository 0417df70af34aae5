// Exact fp32 token scan of the n-step gated DeltaNet, forward and reverse-time backward: the reference's
// "triton" / "ref" scan (archbench/layers/nsgdn.py:80-154, ops :162-216; the recurrence of nsgdn_ref, :408-417).
// Per token t of a (b, h) sequence, with the state S [V, K] fp32 from zero (or from an initial state):
//     S <- e^{la_t} S;   r_t = v_t - S k_t;   S <- S + r_t u_t^T;   y_t = S q_t.
// Rows of S are independent given the token stream.  A workgroup of four waves owns 64 rows; four lanes share a
// row, lane quarter l & 3 holding K / 4 of its entries in registers, so a row's dot products (S k, S q, G u) are a
// partial sum per lane and two DPP steps inside the quad.  k, u, q of a token are workgroup-uniform and reach the
// lanes through LDS (double-buffered: a token is staged while the one before it computes, one barrier per token).
// Every CT tokens the forward stores S (the checkpoint the backward restarts from) in [K][V] order.
// The backward walks the checkpoints in reverse: it recomputes the chunk's states forward from the checkpoint
// (keeping e^{la} S before each token's update in a per-workgroup scratch) and accumulates dq = sum_rows S_t^T dy_t,
// then runs the chunk's tokens backward with the state gradient G [V, K] in registers beside S:
//     G += dy_t q_t^T;  dv_t = G u_t;  du_t = sum_rows G r_t;  G -= dv_t k_t^T;
//     dk_t = -sum_rows (e^{la} S_{t-1}) dv_t;  dla_t = sum (G o e^{la} S_{t-1});  G <- e^{la_t} G.
// Sums over rows are a reduce-scatter over the wave's 16 rows (lane swaps and DPP, no LDS crossbar), then over the
// four waves through LDS (a fixed order, no atomics), then over a head's V / 64 workgroups through partial rows that
// the host adds.
#include <hip/hip_runtime.h>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int TS_CT = 32;                  // tokens between checkpoints
constexpr int TS_ROWS = 64;                // state rows per workgroup
constexpr int TS_THREADS = 4 * TS_ROWS;    // four lanes per row
constexpr int TS_WAVES = TS_THREADS / 64;  // each wave holds 16 rows

// sum over the four lanes of a row (a quad), left in each of them
__device__ __forceinline__ float ts_quad_sum(float x) { return dpp_sum_step<0x4e>(dpp_sum_step<0xb1>(x)); }

// Reduce-scatter over a wave's 16 rows: N values per lane (its quarter's local columns), summed over the 16 lanes
// that share l & 3 (lane bits 2..5).  Lane l ends with the sums of local columns m + (N / 16) (l >> 2), m < N / 16,
// in a[0 .. N / 16).  Each round pairs lanes that differ in one bit and hold the same column set: one keeps the lower
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
  // bit 4: the same with v_permlane16_swap between even and odd 16-lane rows
#pragma unroll
  for (int m = 0; m < N / 4; ++m) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[m]), __float_as_uint(a[m + N / 4]), false, false);
    a[m] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  // bit 3: row_ror:8 pairs lanes p and p ^ 8 of a 16-lane row
  const int b3 = (l >> 3) & 1;
#pragma unroll
  for (int m = 0; m < N / 8; ++m) {
    const float keep = b3 ? a[m + N / 8] : a[m], send = b3 ? a[m] : a[m + N / 8];
    a[m] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0x128, 0xf, 0xf, false));
  }
  // bit 2: lanes l and l ^ 4
  const int b2 = (l >> 2) & 1;
#pragma unroll
  for (int m = 0; m < N / 16; ++m) {
    const float keep = b2 ? a[m + N / 16] : a[m], send = b2 ? a[m] : a[m + N / 16];
    a[m] = keep + __shfl_xor(send, 4);
  }
}

// A token's k, u, q in LDS: per vector four quarter blocks of K / 4 floats, each padded by 4 so that the four lanes
// of a quad (one per block) read different banks with 16-byte reads.  Threads below 3 K / 4 (or the K / 4 of u alone)
// each load one float4 of the next token while the current one computes and store it here when it is done.
template <int K>
struct TokStage {
  static constexpr int KQ = K / 4, LD = KQ + 4, VEC = 4 * LD, SIZE = 3 * VEC;
  f32x4 x;
  __device__ __forceinline__ void load(const float* kp, const float* up, const float* qp, int64_t t, int tid,
                                       bool kq) {
    const int vec = tid / KQ, e4 = tid - vec * KQ;
    if (kq ? tid < 3 * KQ : vec == 1) {
      const float* src = vec == 0 ? kp : vec == 1 ? up : qp;
      x = *reinterpret_cast<const f32x4*>(src + t * K + 4 * e4);
    }
  }
  __device__ __forceinline__ void stage(float* sv, int tid, bool kq) const {
    const int vec = tid / KQ, c = 4 * (tid - vec * KQ), qd = c / KQ;
    if (kq ? tid < 3 * KQ : vec == 1) *reinterpret_cast<f32x4*>(sv + vec * VEC + qd * LD + c - qd * KQ) = x;
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

// grid B * H * NB (NB = ceil(V / 64)) workgroups of 256 threads: workgroup x -> (b h, row block vb)
template <int K>
__global__ __launch_bounds__(TS_THREADS) void token_scan_fwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ u, const float* __restrict__ v,
    const float* __restrict__ la, const float* __restrict__ h0, float* __restrict__ y, float* __restrict__ r,
    float* __restrict__ st, float* __restrict__ hT, int T_, int H, int V, int NCH, int NB) {
  using TS = TokStage<K>;
  constexpr int KQ = TS::KQ;
  __shared__ __attribute__((aligned(16))) float sv[2][TS::SIZE];
  const int tid = threadIdx.x, l = lane_id(), qd = l & 3;
  const int pid = blockIdx.x, bh = pid / NB, vb = pid - bh * NB;
  const int b = bh / H, h = bh - b * H;
  const int vi = vb * TS_ROWS + (tid >> 2);
  const bool on = vi < V;
  const int vc = on ? vi : V - 1;  // rows past V compute on row V-1 and store nothing
  // states [B, H, K, V] (fla's layout): entry (row vi, column qd KQ + j) at cb + j V
  const int64_t cb = (int64_t)bh * K * V + (int64_t)qd * KQ * V + vi;
  float S[KQ];
#pragma unroll
  for (int j = 0; j < KQ; ++j) S[j] = h0 && on ? h0[cb + (int64_t)j * V] : 0.f;
  float* stb = st + (int64_t)bh * NCH * K * V + (int64_t)qd * KQ * V + vi;
  const int64_t tok_first = (int64_t)b * T_ * H + h;
  TS nx;
  nx.load(k, u, q, tok_first, tid, true);  // T_ >= 1 here (the host returns before launching an empty scan)
  nx.stage(sv[0], tid, true);
  float nv = v[tok_first * V + vc], nla = la[tok_first];
  if (T_ > 1) nx.load(k, u, q, tok_first + H, tid, true);
  __syncthreads();
  int64_t tok = tok_first;
  for (int t = 0; t < T_; ++t, tok += H) {
    if (t % TS_CT == 0 && on) {
      const int64_t c = t / TS_CT;
#pragma unroll
      for (int j = 0; j < KQ; ++j) stb[(c * K + j) * V] = S[j];
    }
    const float vcur = nv, a = expf(nla);
    if (t + 1 < T_) {  // stage the next token (loaded one token ago), load the one after it
      nx.stage(sv[(t + 1) & 1], tid, true);
      nv = v[(tok + H) * V + vc];
      nla = la[tok + H];
      if (t + 2 < T_) nx.load(k, u, q, tok + 2 * H, tid, true);
    }
    const float* sk = sv[t & 1] + qd * TS::LD;
    float kk[KQ];
    ts_read<KQ>(sk, kk);
    float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KQ; ++j) {
      S[j] *= a;
      d[j & 3] = fmaf(S[j], kk[j], d[j & 3]);
    }
    const float rr = vcur - ts_quad_sum((d[0] + d[1]) + (d[2] + d[3]));
    float uu[KQ], qq[KQ];
    ts_read<KQ>(sk + TS::VEC, uu);
    ts_read<KQ>(sk + 2 * TS::VEC, qq);
    float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KQ; ++j) {
      S[j] = fmaf(rr, uu[j], S[j]);
      e[j & 3] = fmaf(S[j], qq[j], e[j & 3]);
    }
    const float yy = ts_quad_sum((e[0] + e[1]) + (e[2] + e[3]));
    if (on && qd == 0) r[tok * V + vi] = rr;
    if (on && qd == 1) y[tok * V + vi] = yy;
    __syncthreads();  // this token's vectors read by every lane; the next token's staged
  }
  if (hT && on) {
#pragma unroll
    for (int j = 0; j < KQ; ++j) hT[cb + (int64_t)j * V] = S[j];
  }
}

// The per-token sums over the workgroup's rows: each wave's column sums (after ts_rows_rs) and its dla go to LDS,
// and the step after (behind the token's barrier) adds the four waves in order and stores the partial row.
template <int K>
struct TokSums {
  float col[2][2][TS_WAVES][K];  // [parity][vector][wave][column]
  float sca[2][TS_WAVES];        // [parity][wave]
  // this wave's reduce-scattered sums of local columns (quarter qd) into vector slot s
  template <int KQ>
  __device__ __forceinline__ void put(int par, int s, const float (&a)[KQ], int l) {
    const int w = wave_id(), c0 = (l & 3) * KQ + (KQ / 16) * (l >> 2);
#pragma unroll
    for (int m = 0; m < KQ / 16; ++m) col[par][s][w][c0 + m] = a[m];
  }
  __device__ __forceinline__ float col_sum(int par, int s, int c) const {
    const float(&x)[TS_WAVES][K] = col[par][s];
    return (x[0][c] + x[1][c]) + (x[2][c] + x[3][c]);
  }
  __device__ __forceinline__ float sca_sum(int par) const {
    return (sca[par][0] + sca[par][1]) + (sca[par][2] + sca[par][3]);
  }
};
static_assert(TS_WAVES == 4, "the LDS sums add four waves");

// Partials: gqp, gup, gkp [NB][B*T*H][K], glap [NB][B*T*H]; sc [B*H*NB][TS_CT][K / 4][256] scratch.
template <int K>
__global__ __launch_bounds__(TS_THREADS) void token_scan_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ u, const float* __restrict__ la,
    const float* __restrict__ r, const float* __restrict__ st, const float* __restrict__ gy,
    const float* __restrict__ dhT, float* __restrict__ gv, float* __restrict__ gqp, float* __restrict__ gup,
    float* __restrict__ gkp, float* __restrict__ glap, float* __restrict__ dh0, float* __restrict__ sc, int T_, int H,
    int V, int NCH, int NB, int64_t ntok) {
  using TS = TokStage<K>;
  constexpr int KQ = TS::KQ;
  __shared__ __attribute__((aligned(16))) float sv[2][TS::SIZE];
  __shared__ TokSums<K> sums;
  const int tid = threadIdx.x, l = lane_id(), qd = l & 3;
  const int pid = blockIdx.x, bh = pid / NB, vb = pid - bh * NB;
  const int b = bh / H, h = bh - b * H;
  const int vi = vb * TS_ROWS + (tid >> 2);
  const bool on = vi < V;
  const float* stb = st + (int64_t)bh * NCH * K * V + (int64_t)qd * KQ * V + vi;
  float* scw = sc + (int64_t)pid * TS_CT * KQ * TS_THREADS + tid;
  float* gq_b = gqp + (int64_t)vb * ntok * K;
  float* gu_b = gup + (int64_t)vb * ntok * K;
  float* gk_b = gkp + (int64_t)vb * ntok * K;
  float* gl_b = glap + (int64_t)vb * ntok;
  TS nx;
  float nla = 0.f, nr = 0.f, ngy = 0.f;
  auto fetch_row = [&](int64_t t) {
    nla = la[t];
    nr = on ? r[t * V + vi] : 0.f;
    ngy = on ? gy[t * V + vi] : 0.f;
  };
  // one pass over the tokens tok_at(0 .. n) with the vectors (u alone unless kq) staged a token ahead; body(i, tok,
  // parity) computes token i from sv[parity] with its row scalars in the registers taken before the staging
  int par = 0;
  auto pass = [&](int n, bool kq, auto&& tok_at, auto&& body) {
    nx.load(k, u, q, tok_at(0), tid, kq);
    nx.stage(sv[par & 1], tid, kq);
    fetch_row(tok_at(0));
    if (n > 1) nx.load(k, u, q, tok_at(1), tid, kq);
    __syncthreads();
    for (int i = 0; i < n; ++i, ++par) {
      const float a = expf(nla), rc = nr, gyc = ngy;
      const int64_t tok = tok_at(i);
      if (i + 1 < n) {
        nx.stage(sv[(par + 1) & 1], tid, kq);
        fetch_row(tok_at(i + 1));
        if (i + 2 < n) nx.load(k, u, q, tok_at(i + 2), tid, kq);
      }
      body(i, tok, a, rc, gyc);
      __syncthreads();  // this token's vectors and sums complete; the next token's staged
    }
  };
  const int64_t cb = (int64_t)bh * K * V + (int64_t)qd * KQ * V + vi;  // [B, H, K, V] states, as in the forward
  float G[KQ];
#pragma unroll
  for (int j = 0; j < KQ; ++j) G[j] = dhT && on ? dhT[cb + (int64_t)j * V] : 0.f;
  for (int c = NCH - 1; c >= 0; --c) {
    const int n = min(TS_CT, T_ - c * TS_CT);
    const int64_t tok0 = ((int64_t)b * T_ + (int64_t)c * TS_CT) * H + h;
    {  // recompute the chunk's states from its checkpoint; dq
      float S[KQ];
#pragma unroll
      for (int j = 0; j < KQ; ++j) S[j] = on ? stb[((int64_t)c * K + j) * V] : 0.f;
      int64_t prev = -1;  // the token whose dq sums wait in LDS
      pass(n, false, [&](int i) { return tok0 + (int64_t)i * H; },
           [&](int i, int64_t tok, float a, float rc, float gyc) {
             const int p = par & 1;
             if (prev >= 0 && tid < K) gq_b[prev * K + tid] = sums.col_sum(p ^ 1, 0, tid);
             float uu[KQ];
             ts_read<KQ>(sv[p] + TS::VEC + qd * TS::LD, uu);
             float t[KQ];
#pragma unroll
             for (int j = 0; j < KQ; ++j) {
               S[j] *= a;
               scw[((int64_t)i * KQ + j) * TS_THREADS] = S[j];
               S[j] = fmaf(rc, uu[j], S[j]);
               t[j] = S[j] * gyc;
             }
             ts_rows_rs<KQ>(t, l);
             sums.put(p, 0, t, l);
             prev = tok;
           });
      if (tid < K) gq_b[prev * K + tid] = sums.col_sum((par - 1) & 1, 0, tid);
    }
    int64_t prev = -1;  // the token whose du, dk, dla sums wait in LDS
    auto flush = [&](int p) {
      if (tid < K) gu_b[prev * K + tid] = sums.col_sum(p, 0, tid);
      else if (tid < 2 * K) gk_b[prev * K + tid - K] = sums.col_sum(p, 1, tid - K);
      if (tid == 0) gl_b[prev] = sums.sca_sum(p);
    };
    pass(n, true, [&](int i) { return tok0 + (int64_t)(n - 1 - i) * H; },
         [&](int i, int64_t tok, float a, float rc, float gyc) {
           const int p = par & 1;
           if (prev >= 0) flush(p ^ 1);
           const float* sb = sv[p] + qd * TS::LD;
           float qq[KQ], uu[KQ];
           ts_read<KQ>(sb + 2 * TS::VEC, qq);
           ts_read<KQ>(sb + TS::VEC, uu);
           float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
           for (int j = 0; j < KQ; ++j) {
             G[j] = fmaf(gyc, qq[j], G[j]);
             d[j & 3] = fmaf(G[j], uu[j], d[j & 3]);
           }
           const float gr = ts_quad_sum((d[0] + d[1]) + (d[2] + d[3]));
           if (on && qd == 0) gv[tok * V + vi] = gr;
           float t[KQ];
#pragma unroll
           for (int j = 0; j < KQ; ++j) t[j] = G[j] * rc;
           ts_rows_rs<KQ>(t, l);
           sums.put(p, 0, t, l);
           float kk[KQ], sp[KQ];
           ts_read<KQ>(sb, kk);
           const int ic = n - 1 - i;  // the token's place in the chunk
#pragma unroll
           for (int j = 0; j < KQ; ++j) {
             sp[j] = scw[((int64_t)ic * KQ + j) * TS_THREADS];
             G[j] = fmaf(-gr, kk[j], G[j]);
             t[j] = -sp[j] * gr;
           }
           ts_rows_rs<KQ>(t, l);
           sums.put(p, 1, t, l);
           float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
           for (int j = 0; j < KQ; ++j) e[j & 3] = fmaf(G[j], sp[j], e[j & 3]);
           const float gl = wave_sum64((e[0] + e[1]) + (e[2] + e[3]));
           if (l == 0) sums.sca[p][wave_id()] = gl;
#pragma unroll
           for (int j = 0; j < KQ; ++j) G[j] *= a;
           prev = tok;
         });
    flush((par - 1) & 1);
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
