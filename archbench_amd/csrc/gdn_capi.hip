// extern "C" entry points: argument validation, workspace carve-up and kernel sequencing.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "../../include/gdn_mi355x.h"
#include "gdn_launch.h"

namespace gdn {

static thread_local char g_err[512] = "";

static int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The kernels move rows with 16-byte vector accesses: every array argument must be 16-byte aligned (any hipMalloc
// or torch allocation is; an offset view may not be).
template <typename... P>
static bool misaligned(const P*... p) {
  return ((reinterpret_cast<uintptr_t>(p) & 15) | ...) != 0;
}

size_t chunk_ws_bytes(int B, int T, int H, int K, int V, int dtype, int parts, ChunkWs* carve, void* base,
                      int ns, int hstride) {
  const size_t es = dtype == DT_BF16 ? 2 : 4;
  const size_t NT = (size_t)(T + CH_TOKENS - 1) / CH_TOKENS;
  const size_t BH = (size_t)B * H;
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) -> void* {
    void* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  ChunkWs ws{};
  if (parts & WS_FACT) {
    ws.Tm = take(BH * NT * CH_TRI_ELEMS * es);
    ws.P = take(BH * NT * CH_TRI_ELEMS * es);
    ws.Gc = static_cast<float*>(take(BH * NT * CH_TOKENS * 4));
  }
  if (parts & WS_STATE) {
    // states of every hstride-th chunk of each swept sequence (a segment when ns > 1; segments hold whole pairs)
    const size_t nts = ns > 1 ? NT / ns : NT;
    ws.hs = take(BH * (size_t)(ns > 1 ? ns : 1) * ((nts + hstride - 1) / hstride) * (size_t)K * V * es);
    ws.Rs = take(BH * NT * CH_TOKENS * (size_t)V * es);
  }
  if (parts & WS_GRAD) {
    ws.dhs = take(BH * NT * (size_t)K * V * es);
    ws.dYs = take(BH * NT * CH_TOKENS * (size_t)V * es);
  }
  const size_t seg_states = ns > 1 ? BH * (size_t)ns * K * V * 4 : 0;  // one fp32 state per segment and head
  if ((parts & WS_SEGF) && ns > 1) {
    ws.phi = static_cast<float*>(take(BH * (size_t)ns * K * K * 4));
    ws.sloc = static_cast<float*>(take(seg_states));
    ws.sin = static_cast<float*>(take(seg_states));
  }
  if ((parts & WS_SEGB) && ns > 1) {
    ws.dsloc = static_cast<float*>(take(seg_states));
    ws.dsend = static_cast<float*>(take(seg_states));
  }
  if (carve) {
    if (parts & WS_FACT) {
      carve->Tm = ws.Tm; carve->P = ws.P; carve->Gc = ws.Gc;
    }
    if (parts & WS_STATE) {
      carve->hs = ws.hs; carve->Rs = ws.Rs;
    }
    if (parts & WS_GRAD) {
      carve->dhs = ws.dhs; carve->dYs = ws.dYs;
    }
    if (parts & WS_SEGF) {
      carve->phi = ws.phi; carve->sloc = ws.sloc; carve->sin = ws.sin;
    }
    if (parts & WS_SEGB) {
      carve->dsloc = ws.dsloc; carve->dsend = ws.dsend;
    }
  }
  return off;
}

int segment_count(int B, int T, int H, int K, int V) {
  (void)K;
  if (T <= 0 || T % CH_TOKENS) return 1;
  const int NT = T / CH_TOKENS;
  const int64_t blocks = (int64_t)(V / 64) * B * H;  // sweep workgroups of the unsegmented problem
  const int cus = device_cu_count();
  int ns = 1;
  // double the segments while the sweeps still fit on the device and each segment keeps >= 16 chunks
  while (blocks * ns * 2 <= cus && NT % (2 * ns) == 0 && NT / (2 * ns) >= 16) ns *= 2;
  // the prefix pass and the scan cost about one and a half sweeps of a segment: below four segments they
  // cost more than the parallelism gains
  return ns >= 4 ? ns : 1;
}

int device_cu_count() {
  static int cached[64] = {0};  // concurrent first calls store the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

bool narrow_sweep_blocks(const ChunkArgs& a, int blocks_per_head) {
  // only when the narrow workgroups all run at once, one per CU (two per CU were measured slower than one wide)
  return (int64_t)blocks_per_head * a.B * a.H <= (int64_t)device_cu_count();
}

bool chunk_shape_supported(int K, int V, int dtype) {
  const bool v_ok = V == 64 || V == 128 || V == 256;
  if (dtype == DT_BF16) return (K == 64 || K == 128) && v_ok;
  if (dtype == DT_F32) return K == 64 && (V == 64 || V == 128);
  return false;
}

__global__ void copy_or_zero_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src ? src[i] : 0.f;
}

// Word copy (or zero fill when src is null) as a kernel rather than hipMemcpyAsync / hipMemsetAsync, so that
// callers may capture these calls in a HIP graph.
__global__ void copy_or_zero_words_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src ? src[i] : 0u;
}

static hipError_t copy_or_zero_bytes(const void* src, void* dst, size_t bytes, hipStream_t st) {
  const int64_t n = (int64_t)(bytes / 4);  // every buffer here is a whole number of 32-bit words
  if (!dst || n == 0) return hipSuccess;
  copy_or_zero_words_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(
      static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), n);
  return hipGetLastError();
}

static hipError_t copy_or_zero(const float* src, float* dst, int64_t n, hipStream_t st) {
  if (!dst || n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  copy_or_zero_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(src, dst, n);
  return hipGetLastError();
}


// ---- per-stage event timing (diagnostic; off unless gdn_profile_enable(1) was called) ----
// Process-wide, so that launches from other host threads count too (PyTorch runs a backward pass on its
// autograd thread): one mutex guards the record, taken only while profiling is on.
enum Stage {
  ST_FWD = 0, ST_BWD_RECOMP, ST_BWD_STATE, ST_BWD_INTRA, ST_STEP, ST_FWD_STASH, ST_FACTORS, ST_CONV_FWD,
  ST_CONV_BWD, ST_NORM_FWD, ST_NORM_BWD, ST_GATES_FWD, ST_GATES_BWD, ST_L2_FWD, ST_L2_BWD, ST_CE, ST_PREFIX,
  ST_SEGSCAN, ST_BWD_LOCAL, ST_WD_FWD, ST_WD_BWD, ST_TSCAN_FWD, ST_TSCAN_BWD, ST_COUNT
};
static const char* kStageNames[ST_COUNT] = {"fwd", "bwd_recompute", "bwd_state", "bwd_intra", "step", "fwd_stash",
                                            "factors", "conv_fwd", "conv_bwd", "norm_fwd", "norm_bwd", "gates_fwd", "gates_bwd",
                                            "l2norm_fwd", "l2norm_bwd", "cross_entropy", "prefix", "seg_scan",
                                            "bwd_local", "write_dir_fwd", "write_dir_bwd", "token_scan_fwd",
                                            "token_scan_bwd"};
struct ProfRec { int stage; hipEvent_t a, b; };
struct Prof {
  std::atomic<bool> on{false};
  std::mutex mu;
  ProfRec rec[4096];
  int n = 0;
  hipEvent_t pool[8192];
  int pool_n = 0, pool_used = 0;
};
static Prof g_prof;

static hipEvent_t prof_event() {  // with g_prof.mu held
  if (g_prof.pool_used < g_prof.pool_n) return g_prof.pool[g_prof.pool_used++];
  hipEvent_t e = nullptr;
  if (g_prof.pool_n < 8192 && hipEventCreate(&e) == hipSuccess) {
    g_prof.pool[g_prof.pool_n++] = e;
    g_prof.pool_used++;
  }
  return e;
}

// Runs `launch` and, when profiling is on, brackets it with events on `st`.
template <typename F>
static hipError_t timed(int stage, hipStream_t st, F&& launch) {
  if (!g_prof.on.load(std::memory_order_relaxed)) return launch();
  std::lock_guard<std::mutex> lock(g_prof.mu);
  if (!g_prof.on.load(std::memory_order_relaxed) || g_prof.n >= 4096) return launch();
  ProfRec r{stage, prof_event(), prof_event()};
  if (r.a) (void)hipEventRecord(r.a, st);
  const hipError_t e = launch();
  if (r.b) (void)hipEventRecord(r.b, st);
  if (r.a && r.b) g_prof.rec[g_prof.n++] = r;
  return e;
}

// The chunk kernels are compiled for K in {64, 128}, V in {64, 128, 256} in bf16, and for K = 64, V in {64, 128}
// in fp32 (the fp32 kernels hold whole fp32 tiles in LDS; at K = 128 they would not fit beside the state).
static int shape_error(int K, int V, int dtype) {
  if (dtype == DT_F32 && chunk_shape_supported(K, V, DT_BF16))
    return fail(GDN_ERR_SHAPE, "fp32 chunk kernels are compiled for K=64, V in {64, 128} only; K=%d V=%d runs in "
                "bf16 (pass bf16 q/k/v, e.g. under torch.autocast(dtype=torch.bfloat16) as archbench's trainer does)",
                K, V);
  return fail(GDN_ERR_SHAPE, "chunk kernels not compiled for K=%d V=%d dtype=%d (bf16: K in {64, 128}, "
              "V in {64, 128, 256}; fp32: K=64, V in {64, 128})", K, V, dtype);
}

static int check_common(int B, int T, int H, int K, int V, int dtype) {
  if (dtype != DT_F32 && dtype != DT_BF16) return fail(GDN_ERR_ARG, "dtype code %d is not GDN_DTYPE_F32/BF16", dtype);
  if (B < 0 || T < 0 || H < 0 || K <= 0 || V <= 0)
    return fail(GDN_ERR_ARG, "invalid sizes B=%d T=%d H=%d K=%d V=%d", B, T, H, K, V);
  if ((int64_t)B * T * H * (K > V ? K : V) >= ((int64_t)1 << 31) * 16)
    return fail(GDN_ERR_ARG, "tensor too large for 64-bit indexing plan");
  // the chunk kernels address one chunk's 64 token rows (row stride H*K or H*V) with 32-bit byte offsets
  if ((int64_t)H * (K > V ? K : V) * CH_TOKENS * (dtype == DT_BF16 ? 2 : 4) >= ((int64_t)1 << 31))
    return fail(GDN_ERR_ARG, "H * max(K, V) = %lld too large for a chunk's 32-bit row offsets",
                (long long)H * (K > V ? K : V));
  return GDN_OK;
}

}  // namespace gdn

using namespace gdn;

extern "C" {

int gdn_version(void) { return 200; }  // 0.2.0: row strides in the conv and norm entry points

int gdn_profile_enable(int on) {
  std::lock_guard<std::mutex> lock(g_prof.mu);
  g_prof.on.store(on != 0, std::memory_order_relaxed);
  g_prof.n = 0;
  g_prof.pool_used = 0;
  return GDN_OK;
}

int gdn_profile_read(double* ms_sum, int* launches, int n_stages) {
  g_err[0] = 0;
  if (!ms_sum || !launches || n_stages < ST_COUNT) return fail(GDN_ERR_ARG, "need arrays of %d stages", ST_COUNT);
  for (int i = 0; i < n_stages; ++i) {
    ms_sum[i] = 0.0;
    launches[i] = 0;
  }
  std::lock_guard<std::mutex> lock(g_prof.mu);
  for (int i = 0; i < g_prof.n; ++i) {
    const ProfRec& r = g_prof.rec[i];
    if (hipEventSynchronize(r.b) != hipSuccess) return fail(GDN_ERR_LAUNCH, "event synchronize failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return fail(GDN_ERR_LAUNCH, "event elapsed failed");
    ms_sum[r.stage] += ms;
    launches[r.stage] += 1;
  }
  g_prof.n = 0;
  g_prof.pool_used = 0;
  return GDN_OK;
}

const char* gdn_profile_stage_name(int stage) {
  return (stage >= 0 && stage < ST_COUNT) ? kStageNames[stage] : "";
}

const char* gdn_last_error(void) { return g_err; }

int gdn_supported(int op, int K, int V, int dtype) {
  if (op == 0) return chunk_shape_supported(K, V, dtype) ? 1 : 0;
  if (op == 1) return (dtype == DT_F32 || dtype == DT_BF16) && step_shape_supported(K, V) ? 1 : 0;
  return 0;
}

int gdn_chunk_fwd_ws_bytes(int B, int T, int H, int K, int V, int dtype, size_t* bytes) {
  g_err[0] = 0;
  if (int e = check_common(B, T, H, K, V, dtype)) return e;
  if (!bytes) return fail(GDN_ERR_ARG, "bytes is NULL");
  *bytes = chunk_ws_bytes(B, T, H, K, V, dtype, WS_FACT | WS_SEGF, nullptr, nullptr, segment_count(B, T, H, K, V), 1);
  return GDN_OK;
}

int gdn_chunk_bwd_ws_bytes(int B, int T, int H, int K, int V, int dtype, size_t* bytes) {
  g_err[0] = 0;
  if (int e = check_common(B, T, H, K, V, dtype)) return e;
  if (!bytes) return fail(GDN_ERR_ARG, "bytes is NULL");
  *bytes = chunk_ws_bytes(B, T, H, K, V, dtype, WS_FACT | WS_STATE | WS_GRAD | WS_SEGF | WS_SEGB, nullptr, nullptr,
                          segment_count(B, T, H, K, V), state_stride(V, dtype, false));
  return GDN_OK;
}

static int stash_sizes(int B, int T, int H, int K, int V, int dtype, bool sepu, size_t* stash_bytes,
                       size_t* bwd_ws_bytes) {
  g_err[0] = 0;
  if (int e = check_common(B, T, H, K, V, dtype)) return e;
  if (!stash_bytes || !bwd_ws_bytes) return fail(GDN_ERR_ARG, "stash_bytes or bwd_ws_bytes is NULL");
  const int ns = segment_count(B, T, H, K, V), hs = state_stride(V, dtype, sepu);
  *stash_bytes = chunk_ws_bytes(B, T, H, K, V, dtype, WS_STASH, nullptr, nullptr, ns, hs);
  *bwd_ws_bytes = chunk_ws_bytes(B, T, H, K, V, dtype, WS_GRAD | WS_SEGB, nullptr, nullptr, ns, hs);
  return GDN_OK;
}

int gdn_chunk_stash_bytes(int B, int T, int H, int K, int V, int dtype, size_t* stash_bytes,
                          size_t* bwd_ws_bytes) {
  return stash_sizes(B, T, H, K, V, dtype, false, stash_bytes, bwd_ws_bytes);
}

int gdn_nsgdn_stash_bytes(int B, int T, int H, int K, int V, int dtype, size_t* stash_bytes,
                          size_t* bwd_ws_bytes) {
  return stash_sizes(B, T, H, K, V, dtype, true, stash_bytes, bwd_ws_bytes);
}

}  // extern "C"

namespace gdn {

// Segmented forward, after the chunk factors of the segmented problem `a` (B*ns sequences of T/ns tokens):
// the prefix pass (each segment's state from zero -- the first from h0 -- and the transitions of the middle
// segments), the scan across segments (the state entering each segment), and `a` set up for the main sweep to
// start every segment from its entering state (it writes hT, from each sequence's last segment).
static hipError_t seg_forward_prefix(ChunkArgs& a, const float* h0, int B, int ns) {
  ChunkArgs p = a;
  p.h0 = h0;
  p.hT = a.ws.sloc;
  p.ns = ns;
  hipError_t e = timed(ST_PREFIX, a.stream, [&] { return launch_fwd(p, FWD_PREFIX); });
  if (e == hipSuccess)
    e = timed(ST_SEGSCAN, a.stream, [&] {
      return launch_seg_scan(a.ws.phi, a.ws.sloc, h0, a.ws.sin, nullptr, B, ns, a.H, a.K, a.V, false, a.stream);
    });
  a.h0 = a.ws.sin;
  a.ns = ns;
  return e;
}

// Forward: o and hT, and with `stash` the per-chunk intermediates for gdn_chunk_bwd_stashed.  With write keys u
// (non-null) beta may be null.
static int chunk_fwd_impl(const void* q, const void* k, const void* u, const void* v, const float* g,
                          const float* beta, const float* h0, void* o, float* hT, void* ws, size_t ws_bytes, int B,
                          int T, int H, int K, int V, float scale, int dtype, void* stream, bool stash,
                          bool segments = true) {
  g_err[0] = 0;
  if (int e = check_common(B, T, H, K, V, dtype)) return e;
  if (!chunk_shape_supported(K, V, dtype))
    return shape_error(K, V, dtype);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nstate = (int64_t)B * H * K * V;
  if (B == 0 || H == 0) return GDN_OK;
  if (T == 0) {
    if (copy_or_zero(h0, hT, nstate, st) != hipSuccess) return fail(GDN_ERR_LAUNCH, "state copy launch failed");
    return GDN_OK;
  }
  if (!q || !k || !v || !g || (!beta && !u) || !o) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (u && dtype != DT_BF16) return fail(GDN_ERR_SHAPE, "separate write keys are compiled for bf16 only");
  if (misaligned(q, k, u, v, g, beta, h0, o, hT, ws))
    return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  ChunkArgs a{};
  const int ns = segments ? segment_count(B, T, H, K, V) : 1;
  a.hstride = state_stride(V, dtype, u != nullptr);
  const size_t need = chunk_ws_bytes(B, T, H, K, V, dtype, stash ? WS_STASH : (WS_FACT | WS_SEGF), &a.ws, ws, ns,
                                     a.hstride);
  if (!ws || ws_bytes < need)
    return fail(GDN_ERR_WORKSPACE, "%s of %zu bytes needed, %zu given", stash ? "stash" : "workspace", need,
                ws ? ws_bytes : (size_t)0);
  a.q = q; a.k = k; a.u = u; a.v = v; a.g = g; a.beta = beta; a.h0 = h0; a.o = o; a.hT = hT;
  a.B = B * ns; a.T = T / ns; a.H = H; a.K = K; a.V = V; a.NT = (a.T + CH_TOKENS - 1) / CH_TOKENS;
  a.scale = scale; a.dtype = dtype; a.stream = st;
  hipError_t e = timed(ST_FACTORS, st, [&] { return launch_factors(a); });
  if (e == hipSuccess && ns > 1) e = seg_forward_prefix(a, h0, B, ns);
  if (e == hipSuccess)
    e = stash ? timed(ST_FWD_STASH, st, [&] { return launch_fwd(a, FWD_STASH); })
              : timed(ST_FWD, st, [&] { return launch_fwd(a, FWD_OUT); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "chunk forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

// Backward; without `stashed` the per-chunk intermediates are recomputed first.  With write keys u (non-null)
// du is written apart from dk, and beta / dbeta may be null.
static int chunk_bwd_impl(const void* q, const void* k, const void* u, const void* v, const float* g,
                          const float* beta, const float* h0, const void* dout, const float* dhT, void* dq, void* dk,
                          void* du, void* dv, float* dg, float* dbeta, float* dh0, const void* stash,
                          size_t stash_bytes, void* ws, size_t ws_bytes, int B, int T, int H, int K, int V,
                          float scale, int dtype, void* stream, bool stashed) {
  g_err[0] = 0;
  if (int e = check_common(B, T, H, K, V, dtype)) return e;
  if (!chunk_shape_supported(K, V, dtype))
    return shape_error(K, V, dtype);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nstate = (int64_t)B * H * K * V;
  if (B == 0 || H == 0) return GDN_OK;
  if (T == 0) {
    if (copy_or_zero(dhT, dh0, nstate, st) != hipSuccess) return fail(GDN_ERR_LAUNCH, "state copy launch failed");
    return GDN_OK;
  }
  if (!q || !k || !v || !g || !dout || !dq || !dk || !dv || !dg || (u ? !du : (!beta || !dbeta)))
    return fail(GDN_ERR_ARG, "null input/output pointer");
  if (u && !stashed) return fail(GDN_ERR_ARG, "separate write keys: the backward needs the forward's stash");
  if (u && dtype != DT_BF16) return fail(GDN_ERR_SHAPE, "separate write keys are compiled for bf16 only");
  if (misaligned(q, k, u, v, g, beta, h0, dout, dhT, dq, dk, du, dv, dg, dbeta, dh0, stash, ws))
    return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  ChunkArgs a{};
  const int ns = segment_count(B, T, H, K, V);  // as the forward that filled the stash chose
  a.hstride = state_stride(V, dtype, u != nullptr);
  if (stashed) {
    // the stash is only read (the kernels take it through the same carve-up as the recompute path's workspace)
    const size_t sneed = chunk_ws_bytes(B, T, H, K, V, dtype, WS_STASH, &a.ws, const_cast<void*>(stash), ns,
                                        a.hstride);
    if (!stash || stash_bytes < sneed)
      return fail(GDN_ERR_WORKSPACE, "stash of %zu bytes needed, %zu given", sneed,
                  stash ? stash_bytes : (size_t)0);
  }
  const int parts = stashed ? (WS_GRAD | WS_SEGB) : (WS_FACT | WS_STATE | WS_GRAD | WS_SEGF | WS_SEGB);
  const size_t need = chunk_ws_bytes(B, T, H, K, V, dtype, parts, &a.ws, ws, ns, a.hstride);
  if (!ws || ws_bytes < need)
    return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws ? ws_bytes : (size_t)0);
  a.q = q; a.k = k; a.u = u; a.v = v; a.g = g; a.beta = beta; a.h0 = h0;
  a.dout = dout; a.dhT = dhT; a.dq = dq; a.dk = dk; a.du = du; a.dv = dv; a.dg = dg; a.dbeta = dbeta; a.dh0 = dh0;
  a.B = B * ns; a.T = T / ns; a.H = H; a.K = K; a.V = V; a.NT = (a.T + CH_TOKENS - 1) / CH_TOKENS;
  a.scale = scale; a.dtype = dtype; a.stream = st;
  hipError_t e = hipSuccess;
  if (!stashed) {
    e = timed(ST_FACTORS, st, [&] { return launch_factors(a); });
    ChunkArgs f = a;
    f.hT = nullptr;
    if (e == hipSuccess && ns > 1) e = seg_forward_prefix(f, h0, B, ns);
    if (e == hipSuccess) e = timed(ST_BWD_RECOMP, st, [&] { return launch_fwd(f, FWD_RECOMPUTE); });
  }
  if (e == hipSuccess && ns > 1) {
    // local reverse pass (each segment's entering-state gradient from a zero leaving gradient -- the last from
    // dhT; not the first segment's, which only dh0 would need), then the scan backwards across segments: the
    // gradient w.r.t. the state leaving each segment.  The main reverse sweep then writes dh0 from each
    // sequence's first segment.
    ChunkArgs l = a;
    l.dhT = dhT;
    l.dh0 = a.ws.dsloc;
    l.ns = ns;
    e = timed(ST_BWD_LOCAL, st, [&] { return launch_bwd_state(l, true); });
    if (e == hipSuccess)
      e = timed(ST_SEGSCAN, st, [&] {
        return launch_seg_scan(a.ws.phi, a.ws.dsloc, dhT, a.ws.dsend, nullptr, B, ns, H, K, V, true, st);
      });
    a.dhT = a.ws.dsend;
    a.ns = ns;
  }
  if (e == hipSuccess) e = timed(ST_BWD_STATE, st, [&] { return launch_bwd_state(a, false); });
  if (e == hipSuccess) e = timed(ST_BWD_INTRA, st, [&] { return launch_bwd_intra(a); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "chunk backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

}  // namespace gdn

extern "C" {

int gdn_chunk_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
                  const float* h0, void* o, float* hT, void* ws, size_t ws_bytes, int B, int T, int H, int K,
                  int V, float scale, int dtype, void* stream) {
  return chunk_fwd_impl(q, k, nullptr, v, g, beta, h0, o, hT, ws, ws_bytes, B, T, H, K, V, scale, dtype, stream,
                        false);
}

}  // extern "C"

namespace gdn {

// ---- allocation-free forward ----------------------------------------------------------------------------------
// The chunk-factor workspace of gdn_chunk_fwd_noalloc lives in this file-scope device array: each GPU the library
// runs on holds its own copy (GDN_NOALLOC_SCRATCH_BYTES) from module load to process exit.  Host code never
// passes the array's name to a kernel (on the host it is a stand-in, not a device address): its device address is
// looked up once per device with that device current and kept in g_scratch_ptr.  Nothing in it needs clearing:
// the factors kernel writes every byte the forward sweep then reads.
static __device__ __align__(256) unsigned char scratch[GDN_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];  // per device ordinal

static int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(GDN_ERR_LAUNCH, "no usable current HIP device (ordinal %d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(GDN_ERR_LAUNCH, "scratch symbol lookup on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GDN_OK;
}

}  // namespace gdn

extern "C" {

int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const float* g, const float* beta,
                          const float* h0, void* o, float* hT, int B, int T, int H, int K, int V, float scale,
                          int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = check_common(B, T, H, K, V, dtype)) return e;
  if (!chunk_shape_supported(K, V, dtype)) return shape_error(K, V, dtype);
  const size_t cap = GDN_NOALLOC_SCRATCH_BYTES;
  const size_t one = chunk_ws_bytes(1, T, H, K, V, dtype, WS_FACT, nullptr, nullptr, 1, 1);
  if (one > cap)
    return fail(GDN_ERR_WORKSPACE, "one sequence needs %zu bytes of chunk factors (H * ceil(T/64) = %lld chunks), "
                "more than the %zu-byte scratch of the allocation-free forward; use gdn_chunk_fwd", one,
                (long long)H * ((T + CH_TOKENS - 1) / CH_TOKENS), cap);
  void* ws = nullptr;
  if (int e = scratch_for_current_device(&ws)) return e;
  // As many sequences per launch group as fit; the groups run one after another on the stream, each reusing the
  // scratch.  Splitting the batch moves every pointer by whole sequences, which keeps the 16-byte alignment the
  // kernels need as long as a sequence's g / beta rows (T * H fp32) are a multiple of 16 bytes.
  int nb = (int)std::min<size_t>((size_t)(B > 0 ? B : 1), cap / one);
  while (nb > 1 && chunk_ws_bytes(nb, T, H, K, V, dtype, WS_FACT, nullptr, nullptr, 1, 1) > cap) --nb;
  if (nb < B && ((size_t)T * H * 4) % 16 != 0)
    return fail(GDN_ERR_WORKSPACE, "B=%d sequences need %zu bytes of chunk factors, more than the %zu-byte scratch, "
                "and T * H = %lld is not a multiple of 4, so the batch cannot be split; use gdn_chunk_fwd", B,
                chunk_ws_bytes(B, T, H, K, V, dtype, WS_FACT, nullptr, nullptr, 1, 1), cap, (long long)T * H);
  const size_t es = dtype == DT_BF16 ? 2 : 4;
  const char* cq = static_cast<const char*>(q);
  const char* ck = static_cast<const char*>(k);
  const char* cv = static_cast<const char*>(v);
  char* co = static_cast<char*>(o);
  if (B == 0)  // nothing to compute; the shared checks still run
    return chunk_fwd_impl(q, k, nullptr, v, g, beta, h0, o, hT, ws, cap, 0, T, H, K, V, scale, dtype, stream, false,
                          false);
  for (int b0 = 0; b0 < B; b0 += nb) {
    const int n = B - b0 < nb ? B - b0 : nb;
    const int64_t tok = (int64_t)b0 * T * H;  // token rows before this group
    const int64_t st = (int64_t)b0 * H * K * V;
    const int e = chunk_fwd_impl(cq ? cq + tok * K * es : nullptr, ck ? ck + tok * K * es : nullptr, nullptr,
                                 cv ? cv + tok * V * es : nullptr, g ? g + tok : nullptr,
                                 beta ? beta + tok : nullptr, h0 ? h0 + st : nullptr,
                                 co ? co + tok * V * es : nullptr, hT ? hT + st : nullptr, ws, cap, n, T, H, K, V,
                                 scale, dtype, stream, false, false);
    if (e != GDN_OK) return e;
  }
  return GDN_OK;
}

int gdn_chunk_fwd_stash(const void* q, const void* k, const void* v, const float* g, const float* beta,
                        const float* h0, void* o, float* hT, void* stash, size_t stash_bytes, int B, int T, int H,
                        int K, int V, float scale, int dtype, void* stream) {
  return chunk_fwd_impl(q, k, nullptr, v, g, beta, h0, o, hT, stash, stash_bytes, B, T, H, K, V, scale, dtype,
                        stream, true);
}

int gdn_chunk_bwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
                  const float* h0, const void* dout, const float* dhT, void* dq, void* dk, void* dv, float* dg,
                  float* dbeta, float* dh0, void* ws, size_t ws_bytes, int B, int T, int H, int K, int V,
                  float scale, int dtype, void* stream) {
  return chunk_bwd_impl(q, k, nullptr, v, g, beta, h0, dout, dhT, dq, dk, nullptr, dv, dg, dbeta, dh0, nullptr, 0,
                        ws, ws_bytes, B, T, H, K, V, scale, dtype, stream, false);
}

int gdn_chunk_bwd_stashed(const void* q, const void* k, const void* v, const float* g, const float* beta,
                          const float* h0, const void* dout, const float* dhT, void* dq, void* dk, void* dv,
                          float* dg, float* dbeta, float* dh0, const void* stash, size_t stash_bytes, void* ws,
                          size_t ws_bytes, int B, int T, int H, int K, int V, float scale, int dtype,
                          void* stream) {
  return chunk_bwd_impl(q, k, nullptr, v, g, beta, h0, dout, dhT, dq, dk, nullptr, dv, dg, dbeta, dh0, stash,
                        stash_bytes, ws, ws_bytes, B, T, H, K, V, scale, dtype, stream, true);
}

int gdn_nsgdn_chunk_fwd(const void* q, const void* k, const void* u, const void* v, const float* la,
                        const float* h0, void* y, float* hT, void* stash, size_t stash_bytes, int B, int T, int H,
                        int K, int V, float scale, int dtype, void* stream) {
  if (!u) {
    g_err[0] = 0;
    return fail(GDN_ERR_ARG, "null input/output pointer");
  }
  return chunk_fwd_impl(q, k, u, v, la, nullptr, h0, y, hT, stash, stash_bytes, B, T, H, K, V, scale, dtype,
                        stream, true);
}

int gdn_nsgdn_chunk_bwd(const void* q, const void* k, const void* u, const void* v, const float* la,
                        const float* h0, const void* dy, const float* dhT, void* dq, void* dk, void* du, void* dv,
                        float* dla, float* dh0, const void* stash, size_t stash_bytes, void* ws, size_t ws_bytes,
                        int B, int T, int H, int K, int V, float scale, int dtype, void* stream) {
  if (!u) {
    g_err[0] = 0;
    return fail(GDN_ERR_ARG, "null input/output pointer");
  }
  return chunk_bwd_impl(q, k, u, v, la, nullptr, h0, dy, dhT, dq, dk, du, dv, dla, nullptr, dh0, stash,
                        stash_bytes, ws, ws_bytes, B, T, H, K, V, scale, dtype, stream, true);
}

int gdn_short_conv_bwd_ws_bytes(int B, int T, int D, int W, size_t* bytes) {
  g_err[0] = 0;
  if (B < 0 || T < 0 || D <= 0 || W <= 0) return fail(GDN_ERR_ARG, "invalid sizes B=%d T=%d D=%d W=%d", B, T, D, W);
  if (!bytes) return fail(GDN_ERR_ARG, "bytes is NULL");
  *bytes = conv_ws_bytes(B, T, D, W);
  return GDN_OK;
}

static int conv_check(int B, int T, int D, int64_t ldx, int W, int norm_group, int dtype, const char* ld_name = "ldx") {
  if (dtype != DT_F32 && dtype != DT_BF16) return fail(GDN_ERR_ARG, "dtype code %d is not GDN_DTYPE_F32/BF16", dtype);
  if (B < 0 || T < 0 || D <= 0 || W <= 0 || norm_group < 0)
    return fail(GDN_ERR_ARG, "invalid sizes B=%d T=%d D=%d W=%d norm_group=%d", B, T, D, W, norm_group);
  if (!conv_shape_supported(D, W, norm_group))
    return fail(GDN_ERR_SHAPE, "short conv not compiled for D=%d W=%d norm_group=%d (D %% 4 == 0, W = 4, "
                "norm_group in {0, 64, 128, 256} dividing D)", D, W, norm_group);
  // each lane reads 4 consecutive channels of a token row: rows start on 4-channel boundaries
  if (ldx < D || ldx % 4 != 0)
    return fail(GDN_ERR_ARG, "%s = %lld must be >= D = %d and a multiple of 4", ld_name, (long long)ldx, D);
  if ((int64_t)T * ldx * (dtype == DT_BF16 ? 2 : 4) >= ((int64_t)1 << 31))
    return fail(GDN_ERR_ARG, "T * %s = %lld too large for the conv backward's 32-bit row offsets", ld_name,
                (long long)T * ldx);
  return GDN_OK;
}

int gdn_short_conv_fwd(const void* x, int64_t ldx, const float* w, const float* bias, const void* state_in, void* y,
                       void* state_out, int B, int T, int D, int W, int norm_group, int dtype, void* stream) {
  g_err[0] = 0;
  if (ldx == 0) ldx = D;
  if (int e = conv_check(B, T, D, ldx, W, norm_group, dtype)) return e;
  if (B == 0) return GDN_OK;
  if (T == 0) {
    if (state_out && state_out != state_in) {
      const size_t n = (size_t)B * D * (W - 1) * (dtype == DT_BF16 ? 2 : 4);
      const hipError_t e = copy_or_zero_bytes(state_in, state_out, n, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "conv state copy: %s", hipGetErrorString(e));
    }
    return GDN_OK;
  }
  if (!x || !w || !y) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (state_out && state_out == state_in) return fail(GDN_ERR_ARG, "state_out must not alias state_in");
  if (misaligned(x, w, bias, state_in, y, state_out)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  ConvArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.state_in = state_in; a.y = y; a.state_out = state_out;
  a.B = B; a.T = T; a.D = D; a.ldx = ldx; a.norm_group = norm_group; a.dtype = dtype;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_CONV_FWD, a.stream, [&] { return launch_conv(a, false); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "short conv forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_short_conv_bwd(const void* x, int64_t ldx, const float* w, const float* bias, const void* state_in,
                       const void* dy, void* dx, int64_t lddx, float* dw, float* dbias, void* dstate_in, void* ws,
                       size_t ws_bytes, int B, int T, int D, int W, int norm_group, int dtype, void* stream) {
  g_err[0] = 0;
  if (ldx == 0) ldx = D;
  if (lddx == 0) lddx = D;
  if (int e = conv_check(B, T, D, ldx, W, norm_group, dtype)) return e;
  if (int e = conv_check(B, T, D, lddx, W, norm_group, dtype, "lddx")) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (B == 0 || T == 0) {
    hipError_t e = copy_or_zero_bytes(nullptr, dw, (size_t)D * W * 4, st);
    if (e == hipSuccess) e = copy_or_zero_bytes(nullptr, dbias, (size_t)D * 4, st);
    if (e == hipSuccess)
      e = copy_or_zero_bytes(nullptr, dstate_in, (size_t)B * D * (W - 1) * (dtype == DT_BF16 ? 2 : 4), st);
    if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "short conv zero-fill: %s", hipGetErrorString(e));
    return GDN_OK;
  }
  if (!x || !w || !dy || !dx || !dw) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(x, w, bias, state_in, dy, dx, dw, dbias, dstate_in, ws))
    return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  const size_t need = conv_ws_bytes(B, T, D, W);
  if (!ws || ws_bytes < need)
    return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws ? ws_bytes : (size_t)0);
  ConvArgs a{};
  a.x = x; a.w = w; a.bias = bias; a.state_in = state_in; a.dy = dy; a.dx = dx; a.dstate_in = dstate_in;
  a.dw = dw; a.dbias = dbias; a.ws = ws;
  a.B = B; a.T = T; a.D = D; a.ldx = ldx; a.lddx = lddx; a.norm_group = norm_group; a.dtype = dtype; a.stream = st;
  const hipError_t e = timed(ST_CONV_BWD, st, [&] { return launch_conv(a, true); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "short conv backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

static int norm_check(int64_t rows, int dim, float eps, int dtype) {
  if (dtype != DT_F32 && dtype != DT_BF16) return fail(GDN_ERR_ARG, "dtype code %d is not GDN_DTYPE_F32/BF16", dtype);
  if (rows < 0 || !(eps >= 0.f)) return fail(GDN_ERR_ARG, "invalid rows=%lld eps=%g", (long long)rows, eps);
  if (!norm_shape_supported(dim)) return fail(GDN_ERR_SHAPE, "gated RMSNorm not compiled for dim=%d (64, 128, 256)", dim);
  return GDN_OK;
}

// ldg = 0: contiguous gate rows; otherwise lines of gpl rows ldg elements apart (checked here)
static int gate_layout_check(const void* gate, int64_t ldg, int gpl, int64_t rows, int dim, int dtype) {
  if (!gate || ldg == 0) return GDN_OK;
  const int esz = dtype == DT_BF16 ? 2 : 4;
  if (gpl < 1 || rows % gpl != 0 || ldg < (int64_t)gpl * dim || (ldg * esz) % 16 != 0 || rows >= ((int64_t)1 << 32))
    return fail(GDN_ERR_ARG, "gate layout: ldg = %lld elements must hold gpl = %d rows of %d (and be a multiple of "
                "16 bytes), rows = %lld a multiple of gpl", (long long)ldg, gpl, dim, (long long)rows);
  return GDN_OK;
}

int gdn_gated_rmsnorm_fwd(const void* x, const void* gate, int64_t ldg, int gpl, const float* weight, void* y,
                          int64_t rows, int dim, float eps, int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = norm_check(rows, dim, eps, dtype)) return e;
  if (int e = gate_layout_check(gate, ldg, gpl, rows, dim, dtype)) return e;
  if (rows == 0) return GDN_OK;
  if (!x || !y) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(x, gate, y)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  NormArgs a{};
  a.x = x; a.gate = gate; a.w = weight; a.y = y; a.rows = rows; a.DV = dim; a.dtype = dtype; a.eps = eps;
  a.ldg = ldg; a.gpl = gpl;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_NORM_FWD, a.stream, [&] { return launch_norm(a, false); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "gated RMSNorm forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_gated_rmsnorm_bwd_ws_bytes(int64_t rows, int dim, size_t* bytes) {
  g_err[0] = 0;
  if (int e = norm_check(rows, dim, 0.f, DT_F32)) return e;
  if (!bytes) return fail(GDN_ERR_ARG, "bytes is NULL");
  *bytes = rows ? norm_ws_bytes(rows, dim) : 0;
  return GDN_OK;
}

int gdn_gated_rmsnorm_bwd(const void* x, const void* gate, int64_t ldg, int gpl, const float* weight,
                          const void* dy, void* dx, void* dgate, float* dweight, void* ws, size_t ws_bytes,
                          int64_t rows, int dim, float eps, int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = norm_check(rows, dim, eps, dtype)) return e;
  if (int e = gate_layout_check(gate, ldg, gpl, rows, dim, dtype)) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) {
    if (copy_or_zero_bytes(nullptr, dweight, (size_t)dim * 4, st) != hipSuccess)
      return fail(GDN_ERR_LAUNCH, "gated RMSNorm zero-fill launch failed");
    return GDN_OK;
  }
  if (!x || !dy || !dx || (gate && !dgate)) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(x, gate, dy, dx, dgate, ws)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  const size_t need = norm_ws_bytes(rows, dim);
  if (!ws || ws_bytes < need)
    return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws ? ws_bytes : (size_t)0);
  NormArgs a{};
  a.x = x; a.gate = gate; a.w = weight; a.dy = dy; a.dx = dx; a.dgate = dgate; a.dw = dweight; a.ws = ws;
  a.rows = rows; a.DV = dim; a.dtype = dtype; a.eps = eps; a.ldg = ldg; a.gpl = gpl; a.stream = st;
  const hipError_t e = timed(ST_NORM_BWD, st, [&] { return launch_norm(a, true); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "gated RMSNorm backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_l2norm_fwd(const void* x, void* y, int64_t rows, int dim, float eps, float scale, int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = norm_check(rows, dim, eps, dtype)) return e;
  if (rows == 0) return GDN_OK;
  if (!x || !y) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(x, y)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  NormArgs a{};
  a.x = x; a.y = y; a.rows = rows; a.DV = dim; a.dtype = dtype; a.eps = eps; a.l2 = true; a.scale = scale;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_L2_FWD, a.stream, [&] { return launch_norm(a, false); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "L2 norm forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_l2norm_bwd(const void* x, const void* dy, void* dx, int64_t rows, int dim, float eps, float scale, int dtype,
                   void* stream) {
  g_err[0] = 0;
  if (int e = norm_check(rows, dim, eps, dtype)) return e;
  if (rows == 0) return GDN_OK;
  if (!x || !dy || !dx) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(x, dy, dx)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  NormArgs a{};
  a.x = x; a.dy = dy; a.dx = dx; a.rows = rows; a.DV = dim; a.dtype = dtype; a.eps = eps; a.l2 = true;
  a.scale = scale; a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_L2_BWD, a.stream, [&] { return launch_norm(a, true); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "L2 norm backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_cross_entropy_fwd_bwd(void* logits, const int64_t* target, float* loss, float* lse, const float* dloss,
                              int64_t N, int V, int64_t ld, int64_t ignore_index, int dtype, void* stream) {
  g_err[0] = 0;
  if (dtype != DT_F32 && dtype != DT_BF16) return fail(GDN_ERR_ARG, "dtype code %d is not GDN_DTYPE_F32/BF16", dtype);
  if (N < 0) return fail(GDN_ERR_ARG, "invalid N=%lld", (long long)N);
  if (!ce_shape_supported(V, ld))
    return fail(GDN_ERR_SHAPE, "cross entropy not compiled for V=%d ld=%lld (V %% 8 == 0, ld %% 8 == 0, V <= 65536)",
                V, (long long)ld);
  if (N == 0) return GDN_OK;
  if (!logits || !target || !loss) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(logits)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  CeArgs a{};
  a.logits = logits; a.target = target; a.loss = loss; a.lse = lse; a.dloss = dloss;
  a.N = N; a.ld = ld; a.V = V; a.dtype = dtype; a.ignore_index = ignore_index;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_CE, a.stream, [&] { return launch_ce(a); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "cross entropy launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

static int write_dir_check(int B, int T, int H, int K, int n_steps, int dtype) {
  if (dtype != DT_F32 && dtype != DT_BF16) return fail(GDN_ERR_ARG, "dtype code %d is not GDN_DTYPE_F32/BF16", dtype);
  if (B < 0 || T < 0 || H <= 0 || K <= 0) return fail(GDN_ERR_ARG, "invalid sizes B=%d T=%d H=%d K=%d", B, T, H, K);
  if (!write_dir_supported(K, n_steps))
    return fail(GDN_ERR_SHAPE, "write direction not compiled for K=%d n_steps=%d (K in {64, 128, 256}, "
                "n_steps >= 1)", K, n_steps);
  return GDN_OK;
}

int gdn_write_direction_fwd(const void* k, const float* beta, const float* lam, void* u, int B, int T, int H, int K,
                            int n_steps, int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = write_dir_check(B, T, H, K, n_steps, dtype)) return e;
  if ((int64_t)B * T == 0) return GDN_OK;
  if (!k || !beta || !lam || !u) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(k, u)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  WriteDirArgs a{};
  a.k = k; a.beta = beta; a.lam = lam; a.u = u;
  a.B = B; a.T = T; a.H = H; a.K = K; a.n_steps = n_steps; a.dtype = dtype;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_WD_FWD, a.stream, [&] { return launch_write_dir(a, false); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "write direction forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_write_direction_bwd(const void* k, const float* beta, const float* lam, const void* du, void* dk,
                            float* dbeta, float* dlam, int B, int T, int H, int K, int n_steps, int dtype,
                            void* stream) {
  g_err[0] = 0;
  if (int e = write_dir_check(B, T, H, K, n_steps, dtype)) return e;
  if ((int64_t)B * T == 0) return GDN_OK;
  if (!k || !beta || !lam || !du || !dk || !dbeta || !dlam) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(k, du, dk)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  WriteDirArgs a{};
  a.k = k; a.beta = beta; a.lam = lam; a.du = du; a.dk = dk; a.dbeta = dbeta; a.dlam = dlam;
  a.B = B; a.T = T; a.H = H; a.K = K; a.n_steps = n_steps; a.dtype = dtype;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_WD_BWD, a.stream, [&] { return launch_write_dir(a, true); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "write direction backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

static int token_scan_check(int B, int T, int H, int K, int V) {
  if (B < 0 || T < 0 || H <= 0 || V <= 0) return fail(GDN_ERR_ARG, "invalid sizes B=%d T=%d H=%d V=%d", B, T, H, V);
  if (!token_scan_supported(K)) return fail(GDN_ERR_SHAPE, "token scan not compiled for K=%d (K in {64, 128})", K);
  if ((int64_t)B * H * ((V + 63) / 64) > INT32_MAX) return fail(GDN_ERR_ARG, "grid too large");
  return GDN_OK;
}

int gdn_token_scan_sizes(int B, int T, int H, int K, int V, size_t* st_bytes, size_t* scratch_bytes,
                         int* n_partials) {
  g_err[0] = 0;
  if (int e = token_scan_check(B, T, H, K, V)) return e;
  if (!st_bytes || !scratch_bytes || !n_partials) return fail(GDN_ERR_ARG, "null output pointer");
  const size_t NB = (size_t)(V + 63) / 64, NCH = (size_t)(T + token_scan_ct() - 1) / token_scan_ct();
  *st_bytes = (size_t)B * H * NCH * K * V * 4;
  *scratch_bytes = (size_t)B * H * NB * token_scan_scratch_floats(K) * 4;
  *n_partials = (int)NB;
  return GDN_OK;
}

int gdn_token_scan_fwd(const float* q, const float* k, const float* u, const float* v, const float* la,
                       const float* h0, float* y, float* r, float* st, size_t st_bytes, float* hT, int B, int T, int H,
                       int K, int V, void* stream) {
  size_t need_st = 0, need_sc = 0;
  int nb = 0;
  if (int e = gdn_token_scan_sizes(B, T, H, K, V, &need_st, &need_sc, &nb)) return e;
  if ((int64_t)B * T == 0) return GDN_OK;
  if (!q || !k || !u || !v || !la || !y || !r || !st) return fail(GDN_ERR_ARG, "null input/output pointer");
  // q, k, u are read as 16-byte vectors, and so are the states
  if (misaligned(q, k, u, h0, hT)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  if (st_bytes < need_st) return fail(GDN_ERR_WORKSPACE, "checkpoint buffer %zu bytes, need %zu", st_bytes, need_st);
  TokenScanArgs a{};
  a.q = q; a.k = k; a.u = u; a.v = v; a.la = la; a.h0 = h0; a.y = y; a.r = r; a.st = st; a.hT = hT;
  a.B = B; a.T = T; a.H = H; a.K = K; a.V = V;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_TSCAN_FWD, a.stream, [&] { return launch_token_scan(a, false); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "token scan forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_token_scan_bwd(const float* q, const float* k, const float* u, const float* la, const float* r,
                       const float* st, size_t st_bytes, const float* dy, const float* dhT, float* dv, float* dq_part,
                       float* du_part, float* dk_part, float* dla_part, float* dh0, float* scratch,
                       size_t scratch_bytes, int B, int T, int H, int K, int V, void* stream) {
  size_t need_st = 0, need_sc = 0;
  int nb = 0;
  if (int e = gdn_token_scan_sizes(B, T, H, K, V, &need_st, &need_sc, &nb)) return e;
  if ((int64_t)B * T == 0) return GDN_OK;
  if (!q || !k || !u || !la || !r || !st || !dy || !dv || !dq_part || !du_part || !dk_part || !dla_part || !scratch)
    return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(q, k, u, dhT, dh0)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  if (st_bytes < need_st) return fail(GDN_ERR_WORKSPACE, "checkpoint buffer %zu bytes, need %zu", st_bytes, need_st);
  if (scratch_bytes < need_sc)
    return fail(GDN_ERR_WORKSPACE, "scratch %zu bytes, need %zu", scratch_bytes, need_sc);
  TokenScanArgs a{};
  a.q = q; a.k = k; a.u = u; a.la = la; a.dy = dy; a.dhT = dhT; a.dv = dv; a.dh0 = dh0;
  a.r = const_cast<float*>(r);  // read only here (the forward writes them)
  a.st = const_cast<float*>(st);
  a.dq_part = dq_part; a.du_part = du_part; a.dk_part = dk_part; a.dla_part = dla_part; a.scratch = scratch;
  a.B = B; a.T = T; a.H = H; a.K = K; a.V = V;
  a.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_TSCAN_BWD, a.stream, [&] { return launch_token_scan(a, true); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "token scan backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

static int gates_check(int64_t ntok, int H, int dtype, bool backward = false) {
  if (dtype != DT_F32 && dtype != DT_BF16) return fail(GDN_ERR_ARG, "dtype code %d is not GDN_DTYPE_F32/BF16", dtype);
  if (ntok < 0 || H <= 0) return fail(GDN_ERR_ARG, "invalid sizes ntok=%lld H=%d", (long long)ntok, H);
  if (backward && H > gates_max_heads())
    return fail(GDN_ERR_SHAPE, "gates backward takes at most %d heads, got H=%d", gates_max_heads(), H);
  return GDN_OK;
}

int gdn_gates_fwd(const void* a, const void* b, int64_t lda, const float* A_log, const float* dt_bias,
                  const float* b_bias, float* g, float* beta, int64_t ntok, int H, float beta_scale, float g_min,
                  int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = gates_check(ntok, H, dtype)) return e;
  if (lda != 0 && lda < H) return fail(GDN_ERR_ARG, "lda = %lld is below H = %d", (long long)lda, H);
  if (ntok == 0) return GDN_OK;
  if (!a || !b || !A_log || !g || !beta) return fail(GDN_ERR_ARG, "null input/output pointer");
  GateArgs ga{};
  ga.a = a; ga.b = b; ga.lda = lda; ga.A_log = A_log; ga.dt_bias = dt_bias; ga.b_bias = b_bias; ga.g = g;
  ga.beta = beta; ga.ntok = ntok; ga.H = H; ga.dtype = dtype; ga.beta_scale = beta_scale; ga.g_min = g_min;
  ga.stream = static_cast<hipStream_t>(stream);
  const hipError_t e = timed(ST_GATES_FWD, ga.stream, [&] { return launch_gates(ga, false); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "gates forward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_gates_bwd_ws_bytes(int64_t ntok, int H, size_t* bytes) {
  g_err[0] = 0;
  if (int e = gates_check(ntok, H, DT_F32, true)) return e;
  if (!bytes) return fail(GDN_ERR_ARG, "bytes is NULL");
  *bytes = ntok ? gates_ws_bytes(ntok, H) : 0;
  return GDN_OK;
}

int gdn_gates_bwd(const void* a, const void* b, int64_t lda, const float* A_log, const float* dt_bias,
                  const float* b_bias, const float* dg, const float* dbeta, void* da, void* db, int64_t ldd,
                  float* dA_log, float* ddt_bias, float* db_bias, void* ws, size_t ws_bytes, int64_t ntok, int H,
                  float beta_scale, float g_min, int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = gates_check(ntok, H, dtype, true)) return e;
  if ((lda != 0 && lda < H) || (ldd != 0 && ldd < H))
    return fail(GDN_ERR_ARG, "lda = %lld / ldd = %lld below H = %d", (long long)lda, (long long)ldd, H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (ntok == 0) {
    hipError_t e = copy_or_zero_bytes(nullptr, dA_log, (size_t)H * 4, st);
    if (e == hipSuccess) e = copy_or_zero_bytes(nullptr, ddt_bias, (size_t)H * 4, st);
    if (e == hipSuccess) e = copy_or_zero_bytes(nullptr, db_bias, (size_t)H * 4, st);
    if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "gates zero-fill: %s", hipGetErrorString(e));
    return GDN_OK;
  }
  if (!a || !b || !A_log || !dg || !dbeta || !da || !db) return fail(GDN_ERR_ARG, "null input/output pointer");
  const size_t need = gates_ws_bytes(ntok, H);
  if (!ws || ws_bytes < need)
    return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws ? ws_bytes : (size_t)0);
  GateArgs ga{};
  ga.a = a; ga.b = b; ga.lda = lda; ga.ldd = ldd; ga.A_log = A_log; ga.dt_bias = dt_bias; ga.b_bias = b_bias;
  ga.dg = dg; ga.dbeta = dbeta; ga.da = da; ga.db = db; ga.dA_log = dA_log; ga.ddt_bias = ddt_bias; ga.db_bias = db_bias; ga.ws = ws;
  ga.ntok = ntok; ga.H = H; ga.dtype = dtype; ga.beta_scale = beta_scale; ga.g_min = g_min; ga.stream = st;
  const hipError_t e = timed(ST_GATES_BWD, st, [&] { return launch_gates(ga, true); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "gates backward launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

int gdn_recurrent_step(const void* q, const void* k, const void* v, const float* g, const float* beta,
                       float* state, void* o, int B, int H, int K, int V, float scale, int dtype, void* stream) {
  g_err[0] = 0;
  if (int e = check_common(B, 1, H, K, V, dtype)) return e;
  if (!step_shape_supported(K, V)) return fail(GDN_ERR_SHAPE, "decode step not compiled for K=%d V=%d", K, V);
  if (B == 0 || H == 0) return GDN_OK;
  if (!q || !k || !v || !g || !beta || !state || !o) return fail(GDN_ERR_ARG, "null input/output pointer");
  if (misaligned(q, k, v, g, beta, state, o)) return fail(GDN_ERR_ARG, "array pointer not 16-byte aligned");
  StepArgs a{q, k, v, g, beta, state, o, B, H, K, V, scale, dtype, static_cast<hipStream_t>(stream)};
  const hipError_t e = timed(ST_STEP, a.stream, [&] { return launch_step(a); });
  if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "decode step launch: %s", hipGetErrorString(e));
  return GDN_OK;
}

}  // extern "C"
