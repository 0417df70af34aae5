// Exact fp32 token scan of the n-step gated DeltaNet, forward and reverse-time backward: the reference's
// "triton" / "ref" scan (archbench/layers/nsgdn.py:80-154, ops :162-216; the recurrence of nsgdn_ref, :408-417).
// Per token t of a (b, h) sequence, with the state S [V, K] fp32 from zero (or from an initial state):
//     S <- e^{la_t} S;   r_t = v_t - S k_t;   S <- S + r_t u_t^T;   y_t = S q_t.
// Rows of S are independent given the token stream, so each lane of a wave owns one row (its K entries in
// registers) and the wave walks the tokens; k, u, q and la of a token are wave-uniform (staged through LDS).  Every CT
// tokens the forward stores S (the checkpoint the backward restarts from) in [K][V] order, so a wave's 64 rows
// are one coalesced store per column.
// The backward walks the checkpoints in reverse: it recomputes the chunk's states forward from the checkpoint
// (keeping e^{la} S before each token's update in a per-wave scratch) and accumulates dq = sum_rows S_t^T dy_t, then
// runs the chunk's tokens backward with the state gradient G [V, K] per row:
//     G += dy_t q_t^T;  dv_t = G u_t;  du_t = sum_rows G r_t;  G -= dv_t k_t^T;
//     dk_t = -sum_rows (e^{la} S_{t-1}) dv_t;  dla_t = sum (G o e^{la} S_{t-1});  G <- e^{la_t} G.
// Sums over rows are across the lanes of a wave (a reduce-scatter on DPP and lane shuffles, 32 values at a time)
// and across a head's V / 64 waves through per-wave partial rows that the host adds (fixed order, no atomics).
#include <hip/hip_runtime.h>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int TS_CT = 32;  // tokens between checkpoints

// One reduce-scatter round inside a 16-lane DPP row: values a[0 .. 2N) -> a[0 .. N).  The lane whose bit `hi` is
// clear keeps a[k] and sends a[k + N], its DPP partner (pattern CTRL, which pairs lanes with opposite bits) the
// reverse; each adds the value it receives.
template <int N, int CTRL>
__device__ __forceinline__ void ts_rs_dpp(float* a, int hi) {
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float keep = hi ? a[k + N] : a[k], send = hi ? a[k] : a[k + N];
    a[k] = keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), CTRL, 0xf, 0xf, false));
  }
}
// The same round between lanes l and l ^ 16 (a lane shuffle: the pair sits in different DPP rows)
template <int N>
__device__ __forceinline__ void ts_rs_xor16(float* a, int hi) {
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float keep = hi ? a[k + N] : a[k], send = hi ? a[k] : a[k + N];
    a[k] = keep + __shfl_xor(send, 16);
  }
}

// The sum over the wave's 64 lanes of 32 values per lane; lane l (and l ^ 32) ends with the total of value l & 31.
__device__ __forceinline__ float ts_wave_sum32(float (&a)[32], int l) {
#pragma unroll
  for (int k = 0; k < 32; ++k) a[k] += __shfl_xor(a[k], 32);
  ts_rs_xor16<16>(a, (l >> 4) & 1);
  ts_rs_dpp<8, 0x140>(a, (l >> 3) & 1);  // row_mirror: lane 15 - p
  ts_rs_dpp<4, 0x141>(a, (l >> 2) & 1);  // row_half_mirror: lane 7 - p within the half-row
  ts_rs_dpp<2, 0x4e>(a, (l >> 1) & 1);   // quad_perm [2,3,0,1]: lane p ^ 2
  ts_rs_dpp<1, 0xb1>(a, l & 1);          // quad_perm [1,0,3,2]: lane p ^ 1
  return a[0];
}

// Writes sum over the wave's rows of x[j] * s (j < K) to out[0 .. K) (a partial row of the head's K-vector).
template <int K, typename F>
__device__ __forceinline__ void ts_row_sum_store(F&& term, float* __restrict__ out, int l) {
#pragma unroll
  for (int p = 0; p < K / 32; ++p) {
    float a[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) a[j] = term(32 * p + j);
    const float s = ts_wave_sum32(a, l);
    if (l < 32) out[32 * p + l] = s;
  }
}

// A token's wave-uniform vectors (k, u, q) reach the lanes through LDS: each lane loads K / 64 entries of each for
// the next token while the current one computes, writes them to LDS when the current one is done, and every lane
// reads them back as broadcasts.  (Read directly, as scalar loads issued when needed, each token waited on them:
// 5.2 -> 2.0 ms for the forward at B16 T1024 H4 K128 V256.)
template <int K>
struct TokVecs {
  static constexpr int PL = K / 64;
  float k[PL], u[PL], q[PL];
  __device__ __forceinline__ void load(const float* kp, const float* up, const float* qp, int64_t t, int l, bool kq) {
#pragma unroll
    for (int e = 0; e < PL; ++e) {
      u[e] = up[t * K + PL * l + e];
      if (kq) {
        k[e] = kp[t * K + PL * l + e];
        q[e] = qp[t * K + PL * l + e];
      }
    }
  }
  // with every lane done reading the previous token's (the caller's barrier)
  __device__ __forceinline__ void stage(float (&sv)[3][K], int l, bool kq) const {
#pragma unroll
    for (int e = 0; e < PL; ++e) {
      sv[1][PL * l + e] = u[e];
      if (kq) {
        sv[0][PL * l + e] = k[e];
        sv[2][PL * l + e] = q[e];
      }
    }
    __syncthreads();
  }
};

// grid B * H * NB (NB = ceil(V / 64)), one wave each: workgroup x -> (b h, row block vb)
template <int K>
__global__ __launch_bounds__(64) void token_scan_fwd_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ u, const float* __restrict__ v,
                                                            const float* __restrict__ la, const float* __restrict__ h0,
                                                            float* __restrict__ y, float* __restrict__ r,
                                                            float* __restrict__ st, float* __restrict__ hT, int T_,
                                                            int H, int V, int NCH, int NB) {
  __shared__ __attribute__((aligned(16))) float sv[3][K];  // the token's k, u, q
  const int pid = blockIdx.x, bh = pid / NB, vb = pid - bh * NB;
  const int b = bh / H, h = bh - b * H;
  const int l = lane_id(), vi = vb * 64 + l;
  const bool on = vi < V;
  const int vc = on ? vi : V - 1;  // lanes past V compute on row V-1 and store nothing
  // states [B, H, K, V] (fla's layout): row vi of S is column vi of the head's [K, V] block
  const int64_t hbase = (int64_t)bh * K * V + vi;
  float S[K];
#pragma unroll
  for (int j = 0; j < K; ++j) S[j] = h0 && on ? h0[hbase + (int64_t)j * V] : 0.f;
  float* stb = st + (int64_t)bh * NCH * K * V;
  const int64_t tok_first = (int64_t)b * T_ * H + h;
  TokVecs<K> nx;
  float nv = 0.f, nla = 0.f;
  auto fetch = [&](int64_t t) {
    nx.load(k, u, q, t, l, true);
    nv = v[t * V + vc];
    nla = la[t];
  };
  fetch(tok_first);  // T_ >= 1 here (the host returns before launching an empty scan)
  int64_t tok = tok_first;
  for (int c = 0; c < NCH; ++c) {
    if (on) {
#pragma unroll
      for (int j = 0; j < K; ++j) stb[((int64_t)c * K + j) * V + vi] = S[j];
    }
    const int n = min(TS_CT, T_ - c * TS_CT);
    for (int i = 0; i < n; ++i, tok += H) {
      nx.stage(sv, l, true);
      const float vcur = nv, a = expf(nla);
      fetch(c * TS_CT + i + 1 < T_ ? tok + H : tok);  // the next token's (this one's again at the end)
      float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < K; ++j) {
        S[j] *= a;
        d[j & 3] = fmaf(S[j], sv[0][j], d[j & 3]);
      }
      const float rr = vcur - ((d[0] + d[1]) + (d[2] + d[3]));
      float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < K; ++j) {
        S[j] = fmaf(rr, sv[1][j], S[j]);
        e[j & 3] = fmaf(S[j], sv[2][j], e[j & 3]);
      }
      if (on) {
        r[tok * V + vi] = rr;
        y[tok * V + vi] = (e[0] + e[1]) + (e[2] + e[3]);
      }
      __syncthreads();  // every lane done reading this token's vectors before the next are staged
    }
  }
  if (hT && on) {
#pragma unroll
    for (int j = 0; j < K; ++j) hT[hbase + (int64_t)j * V] = S[j];
  }
}

// Partials: gqp, gup, gkp [NB][B*T*H][K], glap [NB][B*T*H]; sc [B*H*NB][TS_CT][K][64] scratch.
template <int K>
__global__ __launch_bounds__(64) void token_scan_bwd_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ u, const float* __restrict__ la,
    const float* __restrict__ r, const float* __restrict__ st, const float* __restrict__ gy,
    const float* __restrict__ dhT, float* __restrict__ gv, float* __restrict__ gqp, float* __restrict__ gup,
    float* __restrict__ gkp, float* __restrict__ glap, float* __restrict__ dh0, float* __restrict__ sc, int T_, int H,
    int V, int NCH, int NB, int64_t ntok) {
  __shared__ float sG[K * 64];  // G, column-major by lane, while the recompute phase holds S
  __shared__ __attribute__((aligned(16))) float sv[3][K];  // the token's k, u, q
  const int pid = blockIdx.x, bh = pid / NB, vb = pid - bh * NB;
  const int b = bh / H, h = bh - b * H;
  const int l = lane_id(), vi = vb * 64 + l;
  const bool on = vi < V;
  const float* stb = st + (int64_t)bh * NCH * K * V;
  float* scw = sc + (int64_t)pid * TS_CT * K * 64;
  float* gq_b = gqp + (int64_t)vb * ntok * K;
  float* gu_b = gup + (int64_t)vb * ntok * K;
  float* gk_b = gkp + (int64_t)vb * ntok * K;
  float* gl_b = glap + (int64_t)vb * ntok;
  TokVecs<K> nx;
  float nla = 0.f, nr = 0.f, ngy = 0.f;
  auto fetch = [&](int64_t t, bool kq) {
    nx.load(k, u, q, t, l, kq);
    nla = la[t];
    nr = on ? r[t * V + vi] : 0.f;
    ngy = on ? gy[t * V + vi] : 0.f;
  };
  const int64_t hbase = (int64_t)bh * K * V + vi;  // [B, H, K, V] states, as in the forward
#pragma unroll
  for (int j = 0; j < K; ++j) sG[j * 64 + l] = dhT && on ? dhT[hbase + (int64_t)j * V] : 0.f;
  for (int c = NCH - 1; c >= 0; --c) {
    const int n = min(TS_CT, T_ - c * TS_CT);
    const int64_t tok0 = ((int64_t)b * T_ + (int64_t)c * TS_CT) * H + h;
    {  // recompute the chunk's states from its checkpoint; dq
      float S[K];
#pragma unroll
      for (int j = 0; j < K; ++j) S[j] = on ? stb[((int64_t)c * K + j) * V + vi] : 0.f;
      fetch(tok0, false);
      for (int i = 0; i < n; ++i) {
        const int64_t tok = tok0 + (int64_t)i * H;
        nx.stage(sv, l, false);
        const float a = expf(nla), rc = nr, gyc = ngy;
        fetch(i + 1 < n ? tok + H : tok, false);
#pragma unroll
        for (int j = 0; j < K; ++j) {
          S[j] *= a;
          scw[((int64_t)i * K + j) * 64 + l] = S[j];
        }
#pragma unroll
        for (int j = 0; j < K; ++j) S[j] = fmaf(rc, sv[1][j], S[j]);
        ts_row_sum_store<K>([&](int j) { return S[j] * gyc; }, gq_b + tok * K, l);
        __syncthreads();  // every lane done reading this token's vectors
      }
    }
    float G[K];
#pragma unroll
    for (int j = 0; j < K; ++j) G[j] = sG[j * 64 + l];
    fetch(tok0 + (int64_t)(n - 1) * H, true);
    for (int i = n - 1; i >= 0; --i) {
      const int64_t tok = tok0 + (int64_t)i * H;
      nx.stage(sv, l, true);
      const float a = expf(nla), rc = nr, gyc = ngy;
      fetch(i > 0 ? tok - H : tok, true);
      float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < K; ++j) {
        G[j] = fmaf(gyc, sv[2][j], G[j]);
        d[j & 3] = fmaf(G[j], sv[1][j], d[j & 3]);
      }
      const float gr = (d[0] + d[1]) + (d[2] + d[3]);
      if (on) gv[tok * V + vi] = gr;
      ts_row_sum_store<K>([&](int j) { return G[j] * rc; }, gu_b + tok * K, l);
#pragma unroll
      for (int j = 0; j < K; ++j) G[j] = fmaf(-gr, sv[0][j], G[j]);
      const float* sp = scw + (int64_t)i * K * 64 + l;
      ts_row_sum_store<K>([&](int j) { return -sp[j * 64] * gr; }, gk_b + tok * K, l);
      float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < K; ++j) e[j & 3] = fmaf(G[j], sp[j * 64], e[j & 3]);
      const float gl = wave_sum64((e[0] + e[1]) + (e[2] + e[3]));
      if (l == 0) gl_b[tok] = gl;
#pragma unroll
      for (int j = 0; j < K; ++j) G[j] *= a;
      __syncthreads();  // every lane done reading this token's vectors
    }
#pragma unroll
    for (int j = 0; j < K; ++j) sG[j * 64 + l] = G[j];
  }
  // G is now the gradient of the state before the first token: the initial state's
  if (dh0 && on) {
#pragma unroll
    for (int j = 0; j < K; ++j) dh0[hbase + (int64_t)j * V] = sG[j * 64 + l];
  }
}

// ---------------------------------------------------------------------------------------------------------
bool token_scan_supported(int K) { return K == 64 || K == 128; }
int token_scan_ct() { return TS_CT; }

template <int K>
static hipError_t token_scan_k(const TokenScanArgs& a, bool backward) {
  const int NB = (a.V + 63) / 64, NCH = (a.T + TS_CT - 1) / TS_CT;
  const dim3 grid((unsigned)(a.B * a.H * NB));
  if (!backward) {
    token_scan_fwd_kernel<K><<<grid, 64, 0, a.stream>>>(a.q, a.k, a.u, a.v, a.la, a.h0, a.y, a.r, a.st, a.hT, a.T,
                                                        a.H, a.V, NCH, NB);
  } else {
    token_scan_bwd_kernel<K><<<grid, 64, 0, a.stream>>>(a.q, a.k, a.u, a.la, a.r, a.st, a.dy, a.dhT, a.dv,
                                                        a.dq_part, a.du_part, a.dk_part, a.dla_part, a.dh0, a.scratch,
                                                        a.T, a.H, a.V, NCH, NB, (int64_t)a.B * a.T * a.H);
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
