// Short causal depthwise convolution + SiLU (+ optional L2 normalisation per head), forward and backward: the
// ShortConvolution in front of the gated DeltaNet op (archbench/layers/nsgdn.py:420-470, the causal_conv1d
// kernels behind fla's GatedDeltaNet; normalisation of q and k per head as in nsgdn.py:527-528).
//
//   z[t,c] = bias[c] + sum_i w[c,i] x[t - (W-1) + i, c]      (x at t < 0 comes from the conv state)
//   y[t,c] = silu(z[t,c]);  with normalisation over each group of NG channels: y / max(||y||_group, 1e-12)
//
// Layout: y, dy [B, T, D] token-major (channel-last); x and dx [B, T] rows of D channels ldx / lddx elements apart
// (= D, or larger to read or write a column slice of a wider tensor in place); w [D, W] fp32 (used rounded to the
// activation dtype; dw is the fp32 gradient of those rounded taps), bias [D] fp32, conv states
// [B, D, W-1] in the activation dtype (the previous W-1 inputs, oldest first).
// Mapping: one wave per (256 channels, 64-token chunk, b); each lane holds 4 consecutive channels, so every token
// row is one 8-byte (bf16) or 16-byte (fp32) access per lane and a wave covers 512 B / 1 KB contiguous.  The W-1
// inputs before a chunk are re-read (a (W-1)/64 halo).  A normalisation group of NG channels spans NG/4 lanes and
// is reduced with lane shuffles.  HBM-bound: x read once, y written once.
// Backward: each wave recomputes z for its chunk plus W-1 tokens of look-ahead, forms dz and emits dx with a
// W-token delay; dw and dbias are summed per wave into a per-chunk partial and reduced over chunks in a fixed
// order by column_sum_kernel (deterministic, no atomics).
#include <type_traits>

#include "gdn_common.h"
#include "gdn_launch.h"

namespace gdn {

constexpr int CONV_L = 64;  // tokens per wave (the backward without normalisation may take CONV_L_LONG)
// Tokens per wave of the backward without the normalisation when the grid stays large (at least
// CONV_LONG_MIN_WAVES_PER_CU waves per CU): each wave's set-up, look-ahead recompute and dw partial are then
// amortised over twice the tokens (96 -> 86 us at B8 T4096 D2048, 99 -> 91 us at B64 T1024 D1024); on small grids
// the shorter chunks' parallelism wins (23 against 39 us at B2 T200 D512).  With the normalisation 64 throughout
// (at the 65m layer's D = 512, 61 against 70 us with 128).
constexpr int CONV_L_LONG = 128, CONV_LONG_MIN_WAVES_PER_CU = 4;
constexpr int CONV_CPL = 4;  // consecutive channels per lane
constexpr int CONV_CW = 64 * CONV_CPL;  // channels per wave
constexpr int CONV_WAVES = 4;  // waves per workgroup, on adjacent channel blocks of the same chunk
constexpr int CONV_UF = 8;  // token rows per load batch, forward
// token rows of x and of dy per load batch, backward: with the per-group normalisation the smaller batch measured
// faster (fewer registers in flight beside the group sums' longer chain: 109 -> 102 us at B8 T4096 D2048), without
// it the larger one (95 against 102 us)
constexpr int CONV_UB = 8, CONV_UB_NORM = 4;

// CONV_CPL = 4 consecutive channels of one token row as loaded (8 B in bf16, 16 B in fp32), converted at use so
// that a whole batch of loads is in flight at once.  The backward reads x and dy and writes dx once each through
// buffer resources with the nontemporal hint (load_buf_nt / store4_buf_nt: 7-17% faster than ordinary global
// accesses, and 32-bit offsets spare it the 64-bit address arithmetic of a VALU-bound loop); the forward, whose
// workgroups re-read a few halo rows of their neighbours, runs slower with the hint and keeps ordinary loads.
template <typename T>
struct Row4;
template <>
struct Row4<bf16> {
  bf16x4 r;
  __device__ __forceinline__ void load(const bf16* p) { r = *reinterpret_cast<const bf16x4*>(p); }
  // nontemporal buffer read at byte offset off
  __device__ __forceinline__ void load_buf_nt(__amdgpu_buffer_rsrc_t rs, int off) {
    r = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 2));
  }
  __device__ __forceinline__ void get(float (&v)[4]) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = static_cast<float>(r[j]);
  }
};
template <>
struct Row4<float> {
  f32x4 r;
  __device__ __forceinline__ void load(const float* p) { r = *reinterpret_cast<const f32x4*>(p); }
  __device__ __forceinline__ void load_buf_nt(__amdgpu_buffer_rsrc_t rs, int off) {
    r = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2));
  }
  __device__ __forceinline__ void get(float (&v)[4]) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = r[j];
  }
};

template <typename T>
__device__ __forceinline__ void store4(T* p, const float (&v)[4]) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<bf16x4*>(p) =
        bf16x4{static_cast<bf16>(v[0]), static_cast<bf16>(v[1]), static_cast<bf16>(v[2]), static_cast<bf16>(v[3])};
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  }
}
// nontemporal buffer write of 4 consecutive channels at byte offset off
template <typename T>
__device__ __forceinline__ void store4_buf_nt(__amdgpu_buffer_rsrc_t rs, int off, const float (&v)[4]) {
  if constexpr (sizeof(T) == 2) {
    const bf16x4 r{static_cast<bf16>(v[0]), static_cast<bf16>(v[1]), static_cast<bf16>(v[2]), static_cast<bf16>(v[3])};
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, r), rs, off, 0, 2);
  } else {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]}), rs, off, 0, 2);
  }
}
// A tap weight at the activation dtype's precision: the reference's conv runs under bf16 autocast, which casts its
// fp32 weight to bf16 (archbench/layers/nsgdn.py:464); rounding here spares the caller two cast passes each way.
template <typename T>
__device__ __forceinline__ float act_round(float x) {
  if constexpr (sizeof(T) == 2) return static_cast<float>(static_cast<bf16>(x));
  return x;
}
// sum over the NG / CONV_CPL lanes of a normalisation group (aligned runs of lanes), the same value in every lane
template <int NG>
__device__ __forceinline__ float group_sum(float s) {
  return lane_group_sum<NG / CONV_CPL>(s);
}
constexpr float NORM_EPS = 1e-12f;  // F.normalize's eps

template <typename T, int W>
__device__ __forceinline__ void load_window(const T* xl, const T* state_in, int64_t srow, int ldx, int t0,
                                            float (&win)[W - 1][CONV_CPL]) {
  // inputs at t0 - (W-1) .. t0 - 1; negative positions from the conv state (zero if none)
#pragma unroll
  for (int i = 0; i < W - 1; ++i) {
    const int t = t0 - (W - 1) + i;
    if (t >= 0) {
      Row4<T> r;
      r.load(xl + (int64_t)t * ldx);
      r.get(win[i]);
    } else if (state_in) {
#pragma unroll
      for (int j = 0; j < CONV_CPL; ++j) win[i][j] = to_f(state_in[srow + (int64_t)j * (W - 1) + (W - 1) + t]);
    } else {
#pragma unroll
      for (int j = 0; j < CONV_CPL; ++j) win[i][j] = 0.f;
    }
  }
}

// Work items: (part = b * nchunk + chunk, 256-channel block), blocks fastest; wave w of workgroup x takes item
// x * CONV_WAVES + w, so the waves of a workgroup, each independent, cover adjacent channel blocks of the same
// token rows (and, when D has fewer than CONV_WAVES blocks, the next chunk's: no wave idles at D = 256 or 512).
__device__ __forceinline__ bool conv_wave_item(int D, int nparts, int& part, int& cw0) {
  const int ncb = (D + CONV_CW - 1) / CONV_CW;
  const int item = (int)blockIdx.x * CONV_WAVES + __builtin_amdgcn_readfirstlane(wave_id());  // uniform: scalar
  part = item / ncb;
  cw0 = (item - part * ncb) * CONV_CW;
  return part < nparts;
}
// Forward: grid ceil(B * nchunk * ceil(D / CONV_CW) / CONV_WAVES), CONV_WAVES waves.  Rows are loaded in batches
// of CONV_UF with the next batch in flight while the current one is computed; the prefetch of the last batch
// re-reads it (start clamped to t1 - CONV_UF) so every load stays inside the chunk.
template <typename T, int W, int NG>
__global__ __launch_bounds__(64 * CONV_WAVES) void conv_silu_fwd_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           const T* __restrict__ state_in, T* __restrict__ y,
                                                           T* __restrict__ state_out, int Tn, int D, int ldx,
                                                           int nchunk, int nparts) {
  constexpr int CPL = CONV_CPL, U = CONV_UF;
  const int l = lane_id();
  int part, cw0;
  if (!conv_wave_item(D, nparts, part, cw0)) return;  // past the last item (waves never synchronise)
  const int c = cw0 + CPL * l;
  const int b = part / nchunk, ch = part - b * nchunk;
  const int t0 = ch * CONV_L, t1 = min(Tn, t0 + CONV_L);
  const bool on = c < D;
  const int cc = on ? c : 0;  // clamped: lanes past D compute on channel 0 and store nothing
  const T* xl = x + (int64_t)b * Tn * ldx + cc;  // token t of x at xl + t * ldx
  T* yl = y + (int64_t)b * Tn * D + cc;
  const int64_t srow = ((int64_t)b * D + cc) * (W - 1);
  float wk[CPL][W], bk[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
#pragma unroll
    for (int i = 0; i < W; ++i) wk[j][i] = act_round<T>(w[(cc + j) * W + i]);
    bk[j] = bias ? bias[cc + j] : 0.f;
  }
  float win[W - 1][CPL];
  load_window<T, W>(xl, state_in, srow, ldx, t0, win);
  auto step = [&](int t, const Row4<T>& row) {
    float xt[CPL], yt[CPL];
    row.get(xt);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      float z = bk[j] + wk[j][W - 1] * xt[j];
#pragma unroll
      for (int i = 0; i < W - 1; ++i) z += wk[j][i] * win[i][j];
      yt[j] = z * fast_sigmoid(z);
      ss += yt[j] * yt[j];
    }
    if constexpr (NG > 0) {
      const float inv = fast_rcp(fmaxf(sqrtf(group_sum<NG>(ss)), NORM_EPS));
#pragma unroll
      for (int j = 0; j < CPL; ++j) yt[j] *= inv;
    }
    if (on) store4(yl + (int64_t)t * D, yt);
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) win[i][j] = win[i + 1][j];
#pragma unroll
    for (int j = 0; j < CPL; ++j) win[W - 2][j] = xt[j];
  };
  const int nfull = (t1 - t0) / U;
  int t = t0;
  if (nfull > 0) {
    Row4<T> buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) buf[u].load(xl + (int64_t)(t0 + u) * ldx);
    for (int n = 0; n < nfull; ++n, t += U) {
      Row4<T> cur[U];
#pragma unroll
      for (int u = 0; u < U; ++u) cur[u] = buf[u];
      const int tn = min(t + U, t1 - U);
#pragma unroll
      for (int u = 0; u < U; ++u) buf[u].load(xl + (int64_t)(tn + u) * ldx);
#pragma unroll
      for (int u = 0; u < U; ++u) step(t + u, cur[u]);
    }
  }
  for (; t < t1; ++t) {
    Row4<T> row;
    row.load(xl + (int64_t)t * ldx);
    step(t, row);
  }
  // the last W-1 inputs become the new conv state (written by the chunk that holds the sequence end; for
  // Tn < W-1 part of it still comes from the old state, which must not be the same buffer)
  if (state_out && on && t1 == Tn) {
    float last[W - 1][CPL];
    load_window<T, W>(xl, state_in, srow, ldx, Tn, last);
#pragma unroll
    for (int i = 0; i < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) state_out[srow + (int64_t)j * (W - 1) + i] = from_f<T>(last[i][j]);
  }
}

// grid and waves as in the forward; partial sums of dw and dbias per (b, chunk) = part.
// Each wave recomputes z over its chunk plus W-1 tokens of look-ahead, forms dz, and emits dx with a W-1 token
// delay; rows of x and dy are loaded in double-buffered batches (CONV_UB, or CONV_UB_NORM with the normalisation) as
// in the forward.
template <typename T, int W, int NG, int L>
__global__ __launch_bounds__(64 * CONV_WAVES) void conv_silu_bwd_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           const T* __restrict__ state_in,
                                                           const T* __restrict__ dy, T* __restrict__ dx,
                                                           T* __restrict__ dstate_in, float* __restrict__ part_out,
                                                           int Tn, int D, int ldx, int lddx, int nchunk,
                                                           int nparts) {
  constexpr int CPL = CONV_CPL, U = NG > 0 ? CONV_UB_NORM : CONV_UB;
  const int l = lane_id();
  int part, cw0;
  if (!conv_wave_item(D, nparts, part, cw0)) return;  // past the last item (waves never synchronise)
  const int c = cw0 + CPL * l;
  const int b = part / nchunk, ch = part - b * nchunk;
  const int t0 = ch * L, t1 = min(Tn, t0 + L);
  const bool on = c < D;
  const int cc = on ? c : 0;
  const T* xl = x + (int64_t)b * Tn * ldx + cc;
  const int64_t srow = ((int64_t)b * D + cc) * (W - 1);
  // the batch element's rows of x ([Tn] rows ldx apart), dy and dx ([Tn][D]) as buffer resources (uniform base,
  // 32-bit offsets: the host keeps Tn * ldx * sizeof(T) under 2 GiB); token t, this lane's channels at byte
  // offset xoff(t) in x and boff(t) in dy and dx
  const int64_t bbase = (int64_t)b * Tn * D;
  const int bbytes = Tn * D * (int)sizeof(T);
  const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(x + (int64_t)b * Tn * ldx), 0,
                                                    Tn * ldx * (int)sizeof(T), BUF_RSRC_WORD3);
  const auto rdy = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(dy + bbase), 0, bbytes, BUF_RSRC_WORD3);
  const auto rdx = __builtin_amdgcn_make_buffer_rsrc(dx + (int64_t)b * Tn * lddx, 0, Tn * lddx * (int)sizeof(T),
                                                     BUF_RSRC_WORD3);
  auto boff = [&](int t) { return (t * D + cc) * (int)sizeof(T); };
  auto xoff = [&](int t) { return (t * ldx + cc) * (int)sizeof(T); };
  auto dxoff = [&](int t) { return (t * lddx + cc) * (int)sizeof(T); };
  float wk[CPL][W], bk[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
#pragma unroll
    for (int i = 0; i < W; ++i) wk[j][i] = act_round<T>(w[(cc + j) * W + i]);
    bk[j] = bias ? bias[cc + j] : 0.f;
  }
  float win[W - 1][CPL], dzw[W - 1][CPL], dwa[CPL][W], dba[CPL];
  load_window<T, W>(xl, state_in, srow, ldx, t0, win);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    dba[j] = 0.f;
#pragma unroll
    for (int i = 0; i < W; ++i) dwa[j][i] = 0.f;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) dzw[i][j] = 0.f;
  }
  // dx[p] = sum_i w[i] dz[p + W-1 - i]: emitted at s = p + W-1 from dz[s] and the W-1 dz before it (dzw).  This
  // wave emits dx for its own tokens, and for chunk 0 also the state gradient (p = -(W-1) .. -1).
  auto emit = [&](int s, const float (&dz)[CPL], bool have_dz) {
    const int p = s - (W - 1);
    if (p >= t0 || (t0 == 0 && p >= -(W - 1))) {
      float o[CPL];
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        o[j] = have_dz ? wk[j][0] * dz[j] : 0.f;
#pragma unroll
        for (int i = 1; i < W; ++i) o[j] += wk[j][i] * dzw[W - 1 - i][j];
      }
      if (on) {
        if (p >= 0) {
          store4_buf_nt<T>(rdx, dxoff(p), o);
        } else if (dstate_in) {
#pragma unroll
          for (int j = 0; j < CPL; ++j) dstate_in[srow + (int64_t)j * (W - 1) + (W - 1) + p] = from_f<T>(o[j]);
        }
      }
    }
  };
  // own = the chunk's own tokens, which carry dw and dbias (the W-1 look-ahead tokens only feed dx)
  auto step = [&](int s, const Row4<T>& xrow, const Row4<T>& dyrow, auto own) {
    float xs[CPL], ds[CPL], dz[CPL];
    xrow.get(xs);
    dyrow.get(ds);
    float z[CPL], sg[CPL], ysl[CPL], ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      z[j] = bk[j] + wk[j][W - 1] * xs[j];
#pragma unroll
      for (int i = 0; i < W - 1; ++i) z[j] += wk[j][i] * win[i][j];
      sg[j] = fast_sigmoid(z[j]);
      ysl[j] = z[j] * sg[j];
      ss += ysl[j] * ysl[j];
    }
    if constexpr (NG > 0) {
      const float nrm = sqrtf(group_sum<NG>(ss));
      const float inv = fast_rcp(fmaxf(nrm, NORM_EPS));
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) dot += ysl[j] * inv * ds[j];
      dot = group_sum<NG>(dot);
      const bool big = nrm > NORM_EPS;
#pragma unroll
      for (int j = 0; j < CPL; ++j) ds[j] = big ? (ds[j] - ysl[j] * inv * dot) * inv : ds[j] * inv;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) dz[j] = ds[j] * sg[j] * (1.f + z[j] * (1.f - sg[j]));
    if constexpr (decltype(own)::value) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
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
      for (int j = 0; j < CPL; ++j) {
        win[i][j] = win[i + 1][j];
        dzw[i][j] = dzw[i + 1][j];
      }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      win[W - 2][j] = xs[j];
      dzw[W - 2][j] = dz[j];
    }
  };
  using Own = std::true_type;
  using LookAhead = std::false_type;
  const int nfull = (t1 - t0) / U;
  int s = t0;
  if (nfull > 0) {
    Row4<T> bx[U], bd[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bx[u].load_buf_nt(rx, xoff(t0 + u));
      bd[u].load_buf_nt(rdy, boff(t0 + u));
    }
    for (int n = 0; n < nfull; ++n, s += U) {
      Row4<T> cx[U], cd[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        cx[u] = bx[u];
        cd[u] = bd[u];
      }
      const int sn = min(s + U, t1 - U);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        bx[u].load_buf_nt(rx, xoff(sn + u));
        bd[u].load_buf_nt(rdy, boff(sn + u));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) step(s + u, cx[u], cd[u], Own{});
    }
  }
  for (; s < t1; ++s) {
    Row4<T> xr, dr;
    xr.load_buf_nt(rx, xoff(s));
    dr.load_buf_nt(rdy, boff(s));
    step(s, xr, dr, Own{});
  }
  const int send = min(Tn, t1 + W - 1);
  for (; s < send; ++s) {
    Row4<T> xr, dr;
    xr.load_buf_nt(rx, xoff(s));
    dr.load_buf_nt(rdy, boff(s));
    step(s, xr, dr, LookAhead{});
  }
  // past the sequence end dz = 0: flush the remaining dx of the chunk's tail (and of the state when Tn is short)
  for (; s < t1 + W - 1; ++s) {
    const float zero[CPL] = {};
    emit(s, zero, false);
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i)
#pragma unroll
      for (int j = 0; j < CPL; ++j) dzw[i][j] = dzw[i + 1][j];
#pragma unroll
    for (int j = 0; j < CPL; ++j) dzw[W - 2][j] = 0.f;
  }
  if (on) {
    float* row = part_out + (int64_t)part * (D * W + D);  // [dw (D x W) | dbias (D)] of this (b, chunk)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
      for (int i = 0; i < W; ++i) row[(cc + j) * W + i] = dwa[j][i];
      row[D * W + cc + j] = dba[j];
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
size_t conv_ws_bytes(int B, int T, int D, int W) {
  // partial rows of the backward: one per (b, chunk of CONV_L or CONV_L_LONG tokens), at most this many
  const size_t nparts = (size_t)B * ((T + CONV_L - 1) / CONV_L);
  return (nparts * (size_t)(D * W + D) * 4 + 255) & ~size_t(255);
}

bool conv_shape_supported(int D, int W, int norm_group) {
  return D > 0 && D % CONV_CPL == 0 && W == 4 &&
         (norm_group == 0 || ((norm_group == 64 || norm_group == 128 || norm_group == 256) && D % norm_group == 0));
}

// workgroups for every (part, 256-channel block) item, CONV_WAVES items each
static dim3 conv_grid(int D, int nparts) {
  const int64_t items = (int64_t)(D + CONV_CW - 1) / CONV_CW * nparts;
  return dim3((unsigned)((items + CONV_WAVES - 1) / CONV_WAVES));
}

template <typename T, int NG>
static hipError_t conv_fwd_k(const ConvArgs& a) {
  const int nchunk = (a.T + CONV_L - 1) / CONV_L;
  const int nparts = a.B * nchunk;
  conv_silu_fwd_kernel<T, 4, NG><<<conv_grid(a.D, nparts), 64 * CONV_WAVES, 0, a.stream>>>(
      static_cast<const T*>(a.x), a.w, a.bias, static_cast<const T*>(a.state_in), static_cast<T*>(a.y),
      static_cast<T*>(a.state_out), a.T, a.D, (int)a.ldx, nchunk, nparts);
  return hipGetLastError();
}

template <typename T, int NG, int L>
static hipError_t conv_bwd_len(const ConvArgs& a) {
  const int nchunk = (a.T + L - 1) / L;
  const int nparts = a.B * nchunk;
  float* part = static_cast<float*>(a.ws);
  conv_silu_bwd_kernel<T, 4, NG, L><<<conv_grid(a.D, nparts), 64 * CONV_WAVES, 0, a.stream>>>(
      static_cast<const T*>(a.x), a.w, a.bias, static_cast<const T*>(a.state_in), static_cast<const T*>(a.dy),
      static_cast<T*>(a.dx), static_cast<T*>(a.dstate_in), part, a.T, a.D, (int)a.ldx, (int)a.lddx, nchunk,
      nparts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_column_sum(part, nparts, a.D * 4 + a.D, ColumnOut{{a.dw, a.dbias, nullptr}, {a.D * 4, a.D, 0}},
                           a.stream);
}

template <typename T, int NG>
static hipError_t conv_bwd_k(const ConvArgs& a) {
  if constexpr (NG == 0) {
    const int64_t long_waves =
        (int64_t)((a.D + CONV_CW - 1) / CONV_CW) * a.B * ((a.T + CONV_L_LONG - 1) / CONV_L_LONG);
    if (long_waves >= (int64_t)CONV_LONG_MIN_WAVES_PER_CU * device_cu_count())
      return conv_bwd_len<T, NG, CONV_L_LONG>(a);
  }
  return conv_bwd_len<T, NG, CONV_L>(a);
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
