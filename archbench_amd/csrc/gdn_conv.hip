// Short causal depthwise convolution + SiLU (+ optional L2 normalisation per head), forward and backward: the
// ShortConvolution in front of the gated DeltaNet op (archbench/layers/nsgdn.py:420-470, the causal_conv1d
// kernels behind fla's GatedDeltaNet; normalisation of q and k per head as in nsgdn.py:527-528).
//
//   z[t,c] = bias[c] + sum_i w[c,i] x[t - (W-1) + i, c]      (x at t < 0 comes from the conv state)
//   y[t,c] = silu(z[t,c]);  with normalisation over each group of NG channels: y / max(||y||_group, 1e-12)
//
// Layout: x, y, dy, dx [B, T, D] token-major (channel-last), w [D, W] fp32, bias [D] fp32, conv states
// [B, D, W-1] in the activation dtype (the previous W-1 inputs, oldest first).
// Mapping: one wave per (512 channels, 64-token chunk, b); each lane holds 8 consecutive channels, so every token
// row is one 16-byte access per lane and a wave covers 1 KB contiguous.  The W-1 inputs before a chunk are
// re-read (a (W-1)/64 halo).  A normalisation group of NG channels spans NG/8 lanes and is reduced with lane
// shuffles.  HBM-bound: x read once, y written once.
// Backward: each wave recomputes z for its chunk plus W-1 tokens of look-ahead, forms dz and emits dx with a
// W-token delay; dw and dbias are summed per wave into a per-chunk partial and reduced over chunks in a fixed
// order by a second kernel (deterministic, no atomics).
#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int CONV_L = 64;    // tokens per wave
constexpr int CONV_CW = 512;  // channels per wave
constexpr int CONV_UF = 8;    // token rows loaded per batch, forward
constexpr int CONV_UB = 4;    // token rows of x and of dy loaded per batch, backward

// 8 consecutive channels of one token row as loaded (16 B in bf16, 32 B in fp32), converted at use so a batch
// of loads is in flight at once
template <typename T>
struct Row8;
template <>
struct Row8<bf16> {
  bf16x8 r;
  __device__ __forceinline__ void load(const bf16* p) { r = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ void get(float (&v)[8]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(r[j]);
  }
};
template <>
struct Row8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ void get(float (&v)[8]) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = a[j];
      v[4 + j] = b[j];
    }
  }
};

template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  Row8<T> r;
  r.load(p);
  r.get(v);
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = static_cast<bf16>(v[j]);
    *reinterpret_cast<bf16x8*>(p) = r;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}
// sum over the NG/8 lanes of a normalisation group (aligned groups of 1, 2, 4, 8, 16 or 32 lanes)
template <int NG>
__device__ __forceinline__ float group_sum(float s) {
  if constexpr (NG >= 16) s += __shfl_xor(s, 1);
  if constexpr (NG >= 32) s += __shfl_xor(s, 2);
  if constexpr (NG >= 64) s += __shfl_xor(s, 4);
  if constexpr (NG >= 128) s += __shfl_xor(s, 8);
  if constexpr (NG >= 256) s += __shfl_xor(s, 16);
  return s;
}
__device__ __forceinline__ float sigmoidf(float z) { return 1.f / (1.f + __expf(-z)); }
constexpr float NORM_EPS = 1e-12f;  // F.normalize's eps

template <typename T, int W>
__device__ __forceinline__ void load_window(const T* x, const T* state_in, int64_t xrow0, int64_t srow, int D,
                                            int t0, float (&win)[W - 1][8]) {
  // inputs at t0 - (W-1) .. t0 - 1; negative positions from the conv state (zero if none)
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int t = t0 - (W - 1) + i;
    if (t >= 0) {
      load8(x + xrow0 + (int64_t)t * D, win[i]);
    } else if (state_in) {
#pragma unroll
      for (int j = 0; j < 8; ++j) win[i][j] = to_f(state_in[srow + (int64_t)j * (W - 1) + (W - 1) + t]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) win[i][j] = 0.f;
    }
  }
}

// grid (B * nchunk, ceil(D / CONV_CW)), 64 threads
template <typename T, int W, int NG>
__global__ __launch_bounds__(64) void conv_silu_fwd_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           const T* __restrict__ state_in, T* __restrict__ y,
                                                           T* __restrict__ state_out, int Tn, int D, int nchunk) {
  const int l = lane_id();
  const int c = blockIdx.y * CONV_CW + 8 * l;
  const int b = blockIdx.x / nchunk, ch = blockIdx.x - b * nchunk;
  const int t0 = ch * CONV_L, t1 = min(Tn, t0 + CONV_L);
  const bool on = c < D;
  const int cc = on ? c : 0;  // clamped: lanes past D compute on channel 0 and store nothing
  const int64_t xrow0 = (int64_t)b * Tn * D + cc;
  const int64_t srow = ((int64_t)b * D + cc) * (W - 1);
  float wk[8][W], bk[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int i = 0; i < W; ++i) wk[j][i] = w[(cc + j) * W + i];
    bk[j] = bias ? bias[cc + j] : 0.f;
  }
  float win[W - 1][8];
  load_window<T, W>(x, state_in, xrow0, srow, D, t0, win);
  auto step = [&](int t, const Row8<T>& row) {
    float xt[8], yt[8];
    row.get(xt);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float z = bk[j] + wk[j][W - 1] * xt[j];
#pragma unroll
      for (int i = 0; i < W - 1; ++i) z += wk[j][i] * win[i][j];
      yt[j] = z * sigmoidf(z);
      ss += yt[j] * yt[j];
    }
    if constexpr (NG > 0) {
      const float inv = 1.f / fmaxf(sqrtf(group_sum<NG>(ss)), NORM_EPS);
#pragma unroll
      for (int j = 0; j < 8; ++j) yt[j] *= inv;
    }
    if (on) store8(y + xrow0 + (int64_t)t * D, yt);
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) win[i][j] = win[i + 1][j];
#pragma unroll
    for (int j = 0; j < 8; ++j) win[W - 2][j] = xt[j];
  };
  int t = t0;
  for (; t + CONV_UF <= t1; t += CONV_UF) {
    Row8<T> rows[CONV_UF];
#pragma unroll
    for (int u = 0; u < CONV_UF; ++u) rows[u].load(x + xrow0 + (int64_t)(t + u) * D);
#pragma unroll
    for (int u = 0; u < CONV_UF; ++u) step(t + u, rows[u]);
  }
  for (; t < t1; ++t) {
    Row8<T> row;
    row.load(x + xrow0 + (int64_t)t * D);
    step(t, row);
  }
  // the last W-1 inputs become the new conv state (written by the chunk that holds the sequence end; for
  // Tn < W-1 part of it still comes from the old state, which must not be the same buffer)
  if (state_out && on && t1 == Tn) {
    float last[W - 1][8];
    load_window<T, W>(x, state_in, xrow0, srow, D, Tn, last);
#pragma unroll
    for (int i = 0; i < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) state_out[srow + (int64_t)j * (W - 1) + i] = from_f<T>(last[i][j]);
  }
}

// grid (B * nchunk, ceil(D / CONV_CW)), 64 threads; partial sums of dw and dbias per (b, chunk) = blockIdx.x
template <typename T, int W, int NG>
__global__ __launch_bounds__(64) void conv_silu_bwd_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           const T* __restrict__ state_in,
                                                           const T* __restrict__ dy, T* __restrict__ dx,
                                                           T* __restrict__ dstate_in, float* __restrict__ dw_part,
                                                           float* __restrict__ db_part, int Tn, int D, int nchunk) {
  const int l = lane_id();
  const int c = blockIdx.y * CONV_CW + 8 * l;
  const int b = blockIdx.x / nchunk, ch = blockIdx.x - b * nchunk;
  const int t0 = ch * CONV_L, t1 = min(Tn, t0 + CONV_L);
  const bool on = c < D;
  const int cc = on ? c : 0;
  const int64_t xrow0 = (int64_t)b * Tn * D + cc;
  const int64_t srow = ((int64_t)b * D + cc) * (W - 1);
  float wk[8][W], bk[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int i = 0; i < W; ++i) wk[j][i] = w[(cc + j) * W + i];
    bk[j] = bias ? bias[cc + j] : 0.f;
  }
  float win[W - 1][8], dzw[W - 1][8], dwa[8][W], dba[8];
  load_window<T, W>(x, state_in, xrow0, srow, D, t0, win);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    dba[j] = 0.f;
#pragma unroll
    for (int i = 0; i < W; ++i) dwa[j][i] = 0.f;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) dzw[i][j] = 0.f;
  }
  // dx[p] = sum_i w[i] dz[p + W-1 - i]: emitted at s = p + W-1 from dz[s] and the W-1 dz before it (dzw).  This
  // wave emits dx for its own tokens, and for chunk 0 also the state gradient (p = -(W-1) .. -1).
  auto emit = [&](int s, const float (&dz)[8], bool have_dz) {
    const int p = s - (W - 1);
    if (p >= t0 || (t0 == 0 && p >= -(W - 1))) {
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o[j] = have_dz ? wk[j][0] * dz[j] : 0.f;
#pragma unroll
        for (int i = 1; i < W; ++i) o[j] += wk[j][i] * dzw[W - 1 - i][j];
      }
      if (on) {
        if (p >= 0) {
          store8(dx + xrow0 + (int64_t)p * D, o);
        } else if (dstate_in) {
#pragma unroll
          for (int j = 0; j < 8; ++j) dstate_in[srow + (int64_t)j * (W - 1) + (W - 1) + p] = from_f<T>(o[j]);
        }
      }
    }
  };
  // s runs over the chunk and W-1 tokens of look-ahead
  auto step = [&](int s, const Row8<T>& xrow, const Row8<T>& dyrow) {
    float xs[8], ds[8], dz[8];
    xrow.get(xs);
    dyrow.get(ds);
    float z[8], sg[8], ysl[8], ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      z[j] = bk[j] + wk[j][W - 1] * xs[j];
#pragma unroll
      for (int i = 0; i < W - 1; ++i) z[j] += wk[j][i] * win[i][j];
      sg[j] = sigmoidf(z[j]);
      ysl[j] = z[j] * sg[j];
      ss += ysl[j] * ysl[j];
    }
    if constexpr (NG > 0) {
      const float nrm = sqrtf(group_sum<NG>(ss));
      const float inv = 1.f / fmaxf(nrm, NORM_EPS);
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) dot += ysl[j] * inv * ds[j];
      dot = group_sum<NG>(dot);
      const bool big = nrm > NORM_EPS;
#pragma unroll
      for (int j = 0; j < 8; ++j) ds[j] = big ? (ds[j] - ysl[j] * inv * dot) * inv : ds[j] * inv;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) dz[j] = ds[j] * sg[j] * (1.f + z[j] * (1.f - sg[j]));
    if (s < t1) {  // this chunk's own tokens carry dw and dbias
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        dba[j] += dz[j];
        dwa[j][W - 1] += dz[j] * xs[j];
#pragma unroll
        for (int i = 0; i < W - 1; ++i) dwa[j][i] += dz[j] * win[i][j];
      }
    }
    emit(s, dz, true);
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        win[i][j] = win[i + 1][j];
        dzw[i][j] = dzw[i + 1][j];
      }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      win[W - 2][j] = xs[j];
      dzw[W - 2][j] = dz[j];
    }
  };
  const int send = min(Tn, t1 + W - 1);
  int s = t0;
  for (; s + CONV_UB <= send; s += CONV_UB) {
    Row8<T> xr[CONV_UB], dr[CONV_UB];
#pragma unroll
    for (int u = 0; u < CONV_UB; ++u) {
      xr[u].load(x + xrow0 + (int64_t)(s + u) * D);
      dr[u].load(dy + xrow0 + (int64_t)(s + u) * D);
    }
#pragma unroll
    for (int u = 0; u < CONV_UB; ++u) step(s + u, xr[u], dr[u]);
  }
  for (; s < send; ++s) {
    Row8<T> xr, dr;
    xr.load(x + xrow0 + (int64_t)s * D);
    dr.load(dy + xrow0 + (int64_t)s * D);
    step(s, xr, dr);
  }
  // past the sequence end dz = 0: flush the remaining dx of the chunk's tail (and of the state when Tn is short)
  for (; s < t1 + W - 1; ++s) {
    const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    emit(s, zero, false);
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) dzw[i][j] = dzw[i + 1][j];
#pragma unroll
    for (int j = 0; j < 8; ++j) dzw[W - 2][j] = 0.f;
  }
  if (on) {
    const int64_t part = (int64_t)blockIdx.x * D + cc;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int i = 0; i < W; ++i) dw_part[(part + j) * W + i] = dwa[j][i];
      db_part[part + j] = dba[j];
    }
  }
}

// dw[c, i] = sum over the B * nchunk partials in order; dbias likewise.
__global__ __launch_bounds__(256) void conv_param_reduce_kernel(const float* __restrict__ dw_part,
                                                                const float* __restrict__ db_part,
                                                                float* __restrict__ dw, float* __restrict__ db,
                                                                int nparts, int D, int W) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < D * W) {
    float s = 0.f;
    for (int p = 0; p < nparts; ++p) s += dw_part[(int64_t)p * D * W + i];
    dw[i] = s;
  } else if (i < D * W + D && db) {
    const int c = i - D * W;
    float s = 0.f;
    for (int p = 0; p < nparts; ++p) s += db_part[(int64_t)p * D + c];
    db[c] = s;
  }
}

// ---------------------------------------------------------------------------------------------------------
size_t conv_ws_bytes(int B, int T, int D, int W) {
  const size_t nparts = (size_t)B * ((T + CONV_L - 1) / CONV_L);
  return ((nparts * D * W * 4 + 255) & ~size_t(255)) + ((nparts * D * 4 + 255) & ~size_t(255));
}

bool conv_shape_supported(int D, int W, int norm_group) {
  return D > 0 && D % 8 == 0 && W == 4 &&
         (norm_group == 0 || ((norm_group == 64 || norm_group == 128 || norm_group == 256) && D % norm_group == 0));
}

template <typename T, int NG>
static hipError_t conv_fwd_k(const ConvArgs& a) {
  const int nchunk = (a.T + CONV_L - 1) / CONV_L;
  dim3 grid(a.B * nchunk, (a.D + CONV_CW - 1) / CONV_CW);
  conv_silu_fwd_kernel<T, 4, NG><<<grid, 64, 0, a.stream>>>(
      static_cast<const T*>(a.x), a.w, a.bias, static_cast<const T*>(a.state_in), static_cast<T*>(a.y),
      static_cast<T*>(a.state_out), a.T, a.D, nchunk);
  return hipGetLastError();
}

template <typename T, int NG>
static hipError_t conv_bwd_k(const ConvArgs& a) {
  const int nchunk = (a.T + CONV_L - 1) / CONV_L;
  const int nparts = a.B * nchunk;
  float* dw_part = static_cast<float*>(a.ws);
  float* db_part = reinterpret_cast<float*>(static_cast<char*>(a.ws) +
                                            (((size_t)nparts * a.D * 4 * 4 + 255) & ~size_t(255)));
  dim3 grid(nparts, (a.D + CONV_CW - 1) / CONV_CW);
  conv_silu_bwd_kernel<T, 4, NG><<<grid, 64, 0, a.stream>>>(
      static_cast<const T*>(a.x), a.w, a.bias, static_cast<const T*>(a.state_in), static_cast<const T*>(a.dy),
      static_cast<T*>(a.dx), static_cast<T*>(a.dstate_in), dw_part, db_part, a.T, a.D, nchunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  conv_param_reduce_kernel<<<dim3((a.D * 4 + a.D + 255) / 256), 256, 0, a.stream>>>(dw_part, db_part, a.dw,
                                                                                   a.dbias, nparts, a.D, 4);
  return hipGetLastError();
}

template <typename T>
static hipError_t conv_dispatch(const ConvArgs& a, bool backward) {
  switch (a.norm_group) {
    case 0: return backward ? conv_bwd_k<T, 0>(a) : conv_fwd_k<T, 0>(a);
    case 64: return backward ? conv_bwd_k<T, 64>(a) : conv_fwd_k<T, 64>(a);
    case 128: return backward ? conv_bwd_k<T, 128>(a) : conv_fwd_k<T, 128>(a);
    case 256: return backward ? conv_bwd_k<T, 256>(a) : conv_fwd_k<T, 256>(a);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_conv(const ConvArgs& a, bool backward) {
  return a.dtype == DT_BF16 ? conv_dispatch<bf16>(a, backward) : conv_dispatch<float>(a, backward);
}

}  // namespace gdn
