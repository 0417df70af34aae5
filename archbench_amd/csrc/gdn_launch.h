// Host-side launch interface between the C ABI (gdn_capi.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gdn {

enum DType { DT_F32 = 0, DT_BF16 = 1 };

constexpr int CH_TOKENS = 64;  // tokens per chunk (the kernels' CH)
// Tm and P per chunk in HBM: the ten 16 x 16 blocks on and below the diagonal of the 64 x 64 matrix (the six above
// are zero), packed row-block-major, each block 16 rows x 16 columns row-major
constexpr int CH_TRI_ELEMS = 10 * 256;

struct StepArgs {
  const void *q, *k, *v;
  const float *g, *beta;
  float* state;
  void* o;
  int B, H, K, V;
  float scale;
  int dtype;
  hipStream_t stream;
};

// The stash keeps the state entering every chunk (stride 1), or entering every even chunk only (stride 2): then the
// gradient kernel advances each even chunk's state through that chunk itself, S' = gamma_C S + (Kd)^T R, from tiles
// it already holds, for the odd chunk that follows.  Stride 2 needs one more K x V bf16 tile of LDS in the gradient
// kernel, which fits for bf16 with V <= 128 and without separate write keys.
inline int state_stride(int V, int dtype, bool sepu) { return dtype == DT_BF16 && !sepu && V <= 128 ? 2 : 1; }

// Chunk workspace carve-up (chunk-major: [B*H][NT][...]).  All offsets are 256-byte aligned.
// Parts: WS_FACT = {Tm, P, Gc} (the chunk factors kernel), WS_STATE = {hs, Rs} (the stashing forward or the
// recompute sweep), WS_GRAD = {dhs, dYs} (the reverse sweep); the gradient kernel reads Gc, hs, Rs, dhs, dYs.
// hs, Rs, dhs and dYs use the fragment layout of the sweeps' accumulators (store_fragblk).
struct ChunkWs {
  void* Tm;   // [BH][NT][CH_TRI_ELEMS]  (I + A)^-1 per chunk (lower blocks, packed), input dtype
  void* P;    // [BH][NT][CH_TRI_ELEMS]  s (Q K^T) o exp(G_i - G_j), lower triangle incl. diagonal (packed)
  float* Gc;  // [BH][NT][64]       chunk-local cumulative log-decay
  void* hs;   // [BH][ceil(NT / hstride)][K][V]  state entering each chunk (hstride 2: each even chunk)
  void* Rs;   // [BH][NT][64][V]    R = U - W S per chunk
  void* dhs;  // [BH][NT][K][V]     dL/d(state leaving each chunk)
  void* dYs;  // [BH][NT][64][V]    dY = Tm^T dL/dR per chunk (the gradient w.r.t. Y, R = Tm Y)
  // segmented sweeps (WS_SEGF, WS_SEGB; see segment_count), fp32, in the segmented [B*NS, H, ...] layout:
  float* phi;    // [B*NS][H][K][K]  transition of each segment
  float* sloc;   // [B*NS][H][K][V]  state leaving each segment from a zero entering state
  float* sin;    // [B*NS][H][K][V]  state entering each segment
  float* dsloc;  // [B*NS][H][K][V]  gradient w.r.t. the entering state, from a zero leaving gradient
  float* dsend;  // [B*NS][H][K][V]  gradient w.r.t. the state leaving each segment
};

// Separate read and write keys: with u non-null the write (state update, the column side of K K^T and Q K^T, the
// dR term U dS) uses u [B,T,H,K] while the read (K S) keeps k, and the backward writes du apart from dk; beta
// may then be null (row scale 1).  With u null, u = k (the gated delta rule).
struct ChunkArgs {
  const void *q, *k, *v;
  const void* u;  // write keys or null
  const float *g, *beta;
  const float* h0;  // [B,H,K,V] or null
  void* o;          // [B,T,H,V] (forward)
  float* hT;        // [B,H,K,V] or null
  // backward
  const void* dout;   // [B,T,H,V]
  const float* dhT;   // or null
  void *dq, *dk, *dv;
  void* du;  // with u
  float *dg, *dbeta;
  float* dh0;  // or null
  ChunkWs ws;
  int B, T, H, K, V, NT;
  float scale;
  int dtype;
  hipStream_t stream;
  // Segmented sweeps: B counts the segments (B = batch * ns, segment s of sequence b is b * ns + s).  With
  // ns > 1 the main sweeps write hT only from each sequence's last segment and dh0 only from its first, and the
  // prefix pass (local reverse pass) starts each sequence's first (last) segment from h0 (dhT), all at the
  // sequence's own index.
  int ns = 1;
  int hstride = 1;  // state_stride(): the stash holds the state entering every hstride-th chunk
};

// Returns the bytes of the requested parts laid out from `base` and, if `carve` is non-null, sets the pointers
// of those parts (others untouched).
// WS_SEGF = {phi, sloc, sin} and WS_SEGB = {dsloc, dsend} are empty unless ns > 1; the stash holds WS_SEGF (the
// backward reads phi).
enum WsPart { WS_FACT = 1, WS_STATE = 2, WS_GRAD = 4, WS_SEGF = 8, WS_SEGB = 16,
              WS_STASH = WS_FACT | WS_STATE | WS_SEGF };
size_t chunk_ws_bytes(int B, int T, int H, int K, int V, int dtype, int parts, ChunkWs* carve, void* base, int ns,
                      int hstride);

// Segmented sweeps: when the state sweeps would leave most compute units idle ((V/64) B H workgroups) and the
// sequence is long, it is cut into NS equal segments of whole chunks, swept in parallel as the problem
// [B*NS, T/NS, H] (the same memory: a segment of a token-major tensor is contiguous), with the states carried
// across segments by a prefix pass and a small scan (gdn_segscan.hip).  Returns NS (1: not segmented); a pure
// function of the shape and the device's CU count, so a forward and its backward agree.
int segment_count(int B, int T, int H, int K, int V);
// Carry states (reverse = false) or state gradients (reverse = true) across the segments of every (b, h).
hipError_t launch_seg_scan(const float* phi, const float* loc, const float* init, float* outs, float* fin, int B,
                           int NS, int H, int K, int V, bool reverse, hipStream_t stream);
bool chunk_shape_supported(int K, int V, int dtype);
bool step_shape_supported(int K, int V);

// Short causal convolution + SiLU (+ per-group L2 normalisation), gdn_conv.hip.
struct ConvArgs {
  const void* x;          // [B, T] rows of D channels, ldx elements apart (ldx >= D)
  const float* w;         // [D, W]
  const float* bias;      // [D] or null
  const void* state_in;   // [B, D, W-1] or null (zeros)
  void* y;                // [B, T, D] (forward)
  void* state_out;        // [B, D, W-1] or null (forward)
  const void* dy;         // backward
  void* dx;               // [B, T] rows of D channels, lddx elements apart
  void* dstate_in;        // or null
  float *dw, *dbias;      // dbias may be null
  void* ws;
  int B, T, D, norm_group, dtype;
  int64_t ldx, lddx;  // row strides of x and dx (>= D)
  hipStream_t stream;
};
size_t conv_ws_bytes(int B, int T, int D, int W);
bool conv_shape_supported(int D, int W, int norm_group);
hipError_t launch_conv(const ConvArgs& a, bool backward);

// Destinations of consecutive column ranges: columns [0, n[0]) go to p[0], the next n[1] to p[1], the next n[2]
// to p[2]; a null p drops its range.
struct ColumnOut {
  float* p[3];
  int n[3];
};
// out[c] = sum over p < nparts of part[p * ld + c] (c < n[0] + n[1] + n[2]), in a fixed order.
hipError_t launch_column_sum(const float* part, int64_t nparts, int64_t ld, ColumnOut out, hipStream_t stream);

// Gated RMSNorm over rows of DV channels (x, gate, y, dy, dx, dgate [rows, DV] in dtype; gate may be null), or
// with l2 set the scaled L2 normalisation y = scale * x / max(||x||, eps) (no gate, no weight).
struct NormArgs {
  const void* x;
  const void* gate;
  int64_t ldg;     // 0: gate rows contiguous; else lines of gpl gate rows, ldg elements apart
  int gpl;
  const float* w;  // [DV] or null (ones)
  void* y;         // forward
  const void* dy;  // backward
  void *dx, *dgate;
  float* dw;       // [DV] or null
  void* ws;        // backward: norm_ws_bytes
  int64_t rows;
  int DV, dtype;
  float eps;
  bool l2;
  float scale;  // l2 only
  hipStream_t stream;
};
bool norm_shape_supported(int DV);
size_t norm_ws_bytes(int64_t rows, int DV);
hipError_t launch_norm(const NormArgs& a, bool backward);

// Gate functions over [ntok, H] (a, b, da, db in dtype; g, beta, dg, dbeta fp32).
struct GateArgs {
  const void *a, *b;
  int64_t lda, ldd;                       // elements between token rows of a, b / of da, db (0: H, contiguous)
  const float *A_log, *dt_bias, *b_bias;  // [H]; dt_bias, b_bias may be null (zero)
  float *g, *beta;                        // forward
  const float *dg, *dbeta;                // backward
  void *da, *db;
  float *dA_log, *ddt_bias, *db_bias;     // [H]; null = not wanted
  void* ws;                               // backward: gates_ws_bytes
  int64_t ntok;
  int H, dtype;
  float beta_scale, g_min;
  hipStream_t stream;
};
size_t gates_ws_bytes(int64_t ntok, int H);
// The backward stages one tile of per-element gradients in LDS: at most this many heads per token.
int gates_max_heads();
hipError_t launch_gates(const GateArgs& a, bool backward);

// Cross-entropy forward + backward in place on logits rows (gdn_ce.hip).
struct CeArgs {
  void* logits;            // [N, ld] in dtype; overwritten with dloss * (softmax - onehot)
  const int64_t* target;   // [N]
  float* loss;             // [N] per-row loss (0 for ignored rows)
  float* lse;              // [N] or null
  const float* dloss;      // device scalar (gradient of each row's loss) or null (1)
  int64_t N, ld;
  int V, dtype;
  int64_t ignore_index;
  hipStream_t stream;
};
bool ce_shape_supported(int V, int64_t ld);
hipError_t launch_ce(const CeArgs& a);

// Write direction of the n-step family (gdn_writedir.hip): k [B,T,H,K] -> u, and the backward.
struct WriteDirArgs {
  const void* k;
  const float* beta;  // [B, T, H]
  const float* lam;   // [H], the effective lam (after the module's softplus)
  void* u;            // forward
  const void* du;     // backward
  void* dk;
  float *dbeta, *dlam;  // [B, T, H]; dlam per row (summed over rows by the caller)
  int B, T, H, K, n_steps, dtype;
  hipStream_t stream;
};
bool write_dir_supported(int K, int n_steps);
hipError_t launch_write_dir(const WriteDirArgs& a, bool backward);

// Exact fp32 token scan of the n-step family (gdn_tokenscan.hip)
struct TokenScanArgs {
  const float *q, *k, *u, *v, *la;  // [B, T, H, K] x3, [B, T, H, V], [B, T, H]
  const float* h0;                  // [B, H, K, V] or NULL (zero)
  float *y, *r, *st, *hT;           // forward: y, r [B, T, H, V]; st [B H][ceil(T / ct)][K][V]; hT or NULL
  const float *dy, *dhT;            // backward (dhT NULL: zero)
  float *dv, *dq_part, *du_part, *dk_part, *dla_part, *dh0, *scratch;  // partials [NB][B T H][K] ([NB][B T H])
  int B, T, H, K, V;
  hipStream_t stream;
};
bool token_scan_supported(int K);
int token_scan_ct();
size_t token_scan_scratch_floats(int K);  // backward scratch per (b, h, 64-row block)
hipError_t launch_token_scan(const TokenScanArgs& a, bool backward);

// Compute units of the current device (cached per device; 256 if the query fails).
int device_cu_count();
// Whether a state sweep with `blocks_per_head` 32-column blocks per (b, h) runs those narrow blocks (four waves
// each, one wave per SIMD) rather than 64-wide blocks of eight waves: when the narrow grid still fits on the
// device in one round, so that the wide grid would leave CUs idle.
bool narrow_sweep_blocks(const ChunkArgs& a, int blocks_per_head);

hipError_t launch_step(const StepArgs& a);
hipError_t launch_factors(const ChunkArgs& a);                  // Tm, P, Gc
// FWD_OUT: o, hT.  FWD_RECOMPUTE: hs, Rs.  FWD_STASH: both.  FWD_PREFIX: hT from a zero state (into sloc) and
// the transition into phi (the prefix pass of a segmented sweep).
enum FwdMode { FWD_OUT = 0, FWD_RECOMPUTE = 1, FWD_STASH = 2, FWD_PREFIX = 3 };
hipError_t launch_fwd(const ChunkArgs& a, FwdMode mode);
// dhs, dYs, dh0; local (the first pass of a segmented sweep): dh0 only
hipError_t launch_bwd_state(const ChunkArgs& a, bool local);
hipError_t launch_bwd_intra(const ChunkArgs& a);                 // dq, dk, dv, dg, dbeta

}  // namespace gdn
