/* C ABI of the MI355X-native gated DeltaNet (GDN) token-mixing op.
 *
 * Plain pointers and sizes only: no torch or HIP C++ types cross this boundary.  All device pointers are
 * device memory owned by the caller (in practice torch's caching allocator); the library allocates and frees no
 * memory and never synchronises the host (the opt-in profiling calls below create hipEvents and synchronise on
 * them, and only then).  Every call enqueues its kernels on `stream` (a hipStream_t
 * passed as void*; NULL is the default stream) and returns immediately.
 *
 * Every array pointer must be 16-byte aligned (the kernels move rows with 16-byte accesses); any hipMalloc or
 * torch allocation is, an offset view may not be (GDN_ERR_ARG).
 *
 * Layouts (row-major, contiguous):
 *   q, k  [B, T, H, K]      v, o, dout  [B, T, H, V]       (token-major, "head_first = False")
 *   g, beta [B, T, H] fp32  (g = natural-log decay, beta = write strength)
 *   states h0, hT, dh0, dhT, decode state  [B, H, K, V] fp32
 * dtype selects the element type of q, k, v, o, dout, dq, dk, dv: GDN_DTYPE_F32 or GDN_DTYPE_BF16.
 * Gradients dg, dbeta are fp32.
 *
 * Return value: GDN_OK, or a GDN_ERR_* code with a message available from gdn_last_error() (thread-local).
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_OK 0
#define GDN_ERR_ARG 1       /* null pointer, negative size, bad dtype code */
#define GDN_ERR_SHAPE 2     /* (K, V, dtype) combination not compiled in */
#define GDN_ERR_WORKSPACE 3 /* workspace missing or smaller than the *_ws_bytes query */
#define GDN_ERR_LAUNCH 4    /* HIP reported an error while enqueueing */

#define GDN_DTYPE_F32 0
#define GDN_DTYPE_BF16 1

/* Library version (major * 10000 + minor * 100 + patch). */
int gdn_version(void);

/* Message for the last error raised on the calling thread ("" if none). */
const char* gdn_last_error(void);

/* 1 if the chunk (op = 0) or decode-step (op = 1) kernels are compiled for (K, V, dtype), else 0. */
int gdn_supported(int op, int K, int V, int dtype);

/* Workspace sizes (bytes) for gdn_chunk_fwd / gdn_chunk_bwd.  The buffers the reference allocates inside
 * its ops with torch.empty (archbench/layers/nsgdn.py:172-173, :194-197, :335, :343) are carved from this
 * caller-owned block instead. */
int gdn_chunk_fwd_ws_bytes(int B, int T, int H, int K, int V, int dtype, size_t* bytes);
int gdn_chunk_bwd_ws_bytes(int B, int T, int H, int K, int V, int dtype, size_t* bytes);

/* Chunkwise forward: o = GDN(q, k, v, g, beta; h0), optional final state hT.
 * Replaces archbench::nsgdn_chunk_fwd (archbench/layers/nsgdn.py:352-363) for the plain-GDN write vector
 * u = beta k (nsgdn.py:69), i.e. the forward of fla's chunk_gated_delta_rule behind the `gdn` mixer
 * (archbench/layers/fla.py:36-38).  h0 and hT may be NULL (zero initial state / no final state).
 * Any T >= 0 (ragged last chunk handled in-kernel; the reference falls back to DPLR when T % 64 != 0,
 * nsgdn.py:402-403). */
int gdn_chunk_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
                  const float* h0, void* o, float* hT, void* ws, size_t ws_bytes, int B, int T, int H, int K,
                  int V, float scale, int dtype, void* stream);

/* Chunkwise backward: dq, dk, dv, dg, dbeta (and dh0 if non-NULL) for upstream gradients dout and dhT
 * (dhT may be NULL).  Recomputes the chunk factors and chunk states instead of storing them in the forward.
 * Replaces archbench::nsgdn_chunk_bwd (archbench/layers/nsgdn.py:369-382) with the chain rule through
 * u = beta k (nsgdn.py:69) folded in, i.e. the backward of fla's chunk_gated_delta_rule. */
int gdn_chunk_bwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
                  const float* h0, const void* dout, const float* dhT, void* dq, void* dk, void* dv, float* dg,
                  float* dbeta, float* dh0, void* ws, size_t ws_bytes, int B, int T, int H, int K, int V,
                  float scale, int dtype, void* stream);

/* Allocation-free chunkwise forward.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It computes
 * what gdn_chunk_fwd computes, with the same kernels, but takes no workspace: the chunk factors go to a
 * scratch array of GDN_NOALLOC_SCRATCH_BYTES that the library keeps in device memory on each GPU it runs on
 * (until the process ends).  The results equal gdn_chunk_fwd's bit for bit where gdn_chunk_fwd does not segment
 * its sweeps (long T with few B * H: there it splits each sequence into segments and this entry point does not,
 * and the two agree within rounding).  The call allocates and frees nothing.  Limit: one sequence's factors,
 * H * ceil(T/64) chunks of 10,496 bytes (bf16; 20,736 in fp32), must fit in the scratch; larger batches run as
 * consecutive groups of sequences on `stream` (this needs T * H to be a multiple of 4), otherwise
 * GDN_ERR_WORKSPACE.  Every call on one GPU shares that GPU's scratch, so calls that overlap in time on one GPU
 * (concurrent streams, or several host threads) race and give wrong results: serialise them.  The stream must
 * belong to the calling thread's current device. */
#define GDN_NOALLOC_SCRATCH_BYTES ((size_t)80 << 20)
int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const float* g, const float* beta,
                          const float* h0, void* o, float* hT, int B, int T, int H, int K, int V, float scale,
                          int dtype, void* stream);

/* Training pair.  gdn_chunk_fwd_stash computes what gdn_chunk_fwd computes and also writes into `stash` the
 * per-chunk intermediates the backward needs (chunk factors, chunk-local decay, R = U - W S, and the state
 * entering chunks: in bf16 with V <= 128 only every second chunk's, the backward advancing the state through the
 * chunk between itself; otherwise every chunk's); gdn_chunk_bwd_stashed, called later with the same inputs and the
 * same stash (unchanged in between; it is only read), is gdn_chunk_bwd without its recompute sweep, with `ws`
 * holding only the gradient part of the workspace.  gdn_chunk_stash_bytes gives both sizes.  The reference's
 * forward likewise returns its chunk factor A and cumulative decay g for the backward to reuse
 * (nsgdn.py:352-363, saved at :385-388); keeping states too trades stash_bytes of device memory for one sweep
 * over the sequence. */
int gdn_chunk_stash_bytes(int B, int T, int H, int K, int V, int dtype, size_t* stash_bytes, size_t* bwd_ws_bytes);
int gdn_chunk_fwd_stash(const void* q, const void* k, const void* v, const float* g, const float* beta,
                        const float* h0, void* o, float* hT, void* stash, size_t stash_bytes, int B, int T, int H,
                        int K, int V, float scale, int dtype, void* stream);
int gdn_chunk_bwd_stashed(const void* q, const void* k, const void* v, const float* g, const float* beta,
                          const float* h0, const void* dout, const float* dhT, void* dq, void* dk, void* dv,
                          float* dg, float* dbeta, float* dh0, const void* stash, size_t stash_bytes, void* ws,
                          size_t ws_bytes, int B, int T, int H, int K, int V, float scale, int dtype,
                          void* stream);

/* The same chunk pipeline with separate read and write vectors (the n-step GDN family, archbench's `nsgdn`
 * mixer): per token
 *   S~ = e^la S,   r = v - S~^T k,   S = S~ + u r^T,   y = S^T (scale q)
 * (nsgdn_ref, archbench/layers/nsgdn.py:408-417; the chunked form nsgdn.py:240-249 with
 * L_ij = (k_i . u_j) gamma_i / gamma_j).  Replaces the custom ops archbench::nsgdn_chunk_fwd / _bwd
 * (nsgdn.py:352-397): the reference's forward returns (y, g, A) for its backward, this one fills a stash of
 * gdn_nsgdn_stash_bytes (the state entering every chunk is kept); the backward reads it and writes dq, dk, du,
 * dv, dla (and dh0), with a workspace of the second size gdn_nsgdn_stash_bytes gives.  u has
 * q's shape and dtype; la (natural-log decay) [B,T,H] fp32; h0, hT, dhT, dh0 as for the chunk op (optional);
 * the reference calls it with scale 1 (q pre-scaled) and no states.  bf16 only (as the reference's op, which
 * casts to bf16, nsgdn.py:400-405); K and V as for the chunk op. */
int gdn_nsgdn_stash_bytes(int B, int T, int H, int K, int V, int dtype, size_t* stash_bytes, size_t* bwd_ws_bytes);
int gdn_nsgdn_chunk_fwd(const void* q, const void* k, const void* u, const void* v, const float* la,
                        const float* h0, void* y, float* hT, void* stash, size_t stash_bytes, int B, int T, int H,
                        int K, int V, float scale, int dtype, void* stream);
int gdn_nsgdn_chunk_bwd(const void* q, const void* k, const void* u, const void* v, const float* la,
                        const float* h0, const void* dy, const float* dhT, void* dq, void* dk, void* du, void* dv,
                        float* dla, float* dh0, const void* stash, size_t stash_bytes, void* ws, size_t ws_bytes,
                        int B, int T, int H, int K, int V, float scale, int dtype, void* stream);

/* One recurrent decode step, state updated in place:
 *   r = beta (v - e^g S^T k),  S <- e^g S + k r^T,  o = S^T (scale q)
 * q, k [B, H, K], v, o [B, H, V], g, beta [B, H] fp32, state [B, H, K, V] fp32.
 * The per-token body of the reference's token scan (archbench/layers/nsgdn.py:95-106 and nsgdn_ref,
 * nsgdn.py:413-416), i.e. fla's fused_recurrent_gated_delta_rule at T = 1 with an in-place state. */
int gdn_recurrent_step(const void* q, const void* k, const void* v, const float* g, const float* beta,
                       float* state, void* o, int B, int H, int K, int V, float scale, int dtype, void* stream);

/* Short causal depthwise convolution + SiLU in front of the op, optionally followed by an L2 normalisation over
 * each group of norm_group channels (one head of q or k):
 *   z[t,c] = bias[c] + sum_i w[c,i] x[t-(W-1)+i, c],   y = silu(z),   y <- y / max(||y||_group, 1e-12).
 * Replaces the ShortConv + causal_conv1d custom ops archbench::causal_conv_silu / _bwd
 * (archbench/layers/nsgdn.py:420-470; fla's ShortConvolution in GatedDeltaNet) and the per-head normalisation
 * of q and k (nsgdn.py:527-528).  y, dy [B, T, D] token-major in dtype; x and dx [B, T] rows of D channels ldx /
 * lddx elements apart (D, or 0, when contiguous; larger to read x from, or write dx into, a column slice of a
 * wider [B, T, ld] tensor such as the output of a fused input projection or its gradient; a multiple of 4);
 * w [D, W] and bias [D] fp32 (bias may be NULL); the taps are used rounded to dtype, as the reference's conv runs
 * its weight under bf16 autocast (nsgdn.py:464), and dw is the fp32 gradient of the rounded taps; conv states
 * [B, D, W-1] in dtype, the previous W-1 inputs oldest
 * first (state_in NULL = zeros; state_out NULL = not returned; it must not alias state_in).  Compiled for W = 4,
 * D % 4 == 0, norm_group in {0 (none), 64, 128, 256}.
 * The backward writes dx, dw [D, W] fp32, dbias [D] fp32 (if non-NULL) and dstate_in (if non-NULL); its
 * workspace holds per-chunk partial sums of dw, reduced in a fixed order (deterministic). */
int gdn_short_conv_fwd(const void* x, int64_t ldx, const float* w, const float* bias, const void* state_in, void* y,
                       void* state_out, int B, int T, int D, int W, int norm_group, int dtype, void* stream);
int gdn_short_conv_bwd_ws_bytes(int B, int T, int D, int W, size_t* bytes);
int gdn_short_conv_bwd(const void* x, int64_t ldx, const float* w, const float* bias, const void* state_in,
                       const void* dy, void* dx, int64_t lddx, float* dw, float* dbias, void* dstate_in, void* ws,
                       size_t ws_bytes, int B, int T, int D, int W, int norm_group, int dtype, void* stream);

/* Gated RMSNorm of the op's output, per row of `dim` channels (one head of one token):
 *   y = x * rsqrt(mean(x^2) + eps) * weight * silu(gate)
 * Replaces the output normalisation of the mixer: fla's FusedRMSNormGated in GatedDeltaNet and the reference's
 * self.norm(y) followed by y * F.silu(g) (archbench/layers/nsgdn.py:539-541), as one pass (fp32 arithmetic).
 * x, y, dy, dx, dgate [rows, dim] in dtype; gate may be NULL (plain RMSNorm; dgate unused); weight [dim]
 * fp32 or NULL (ones).  dim in {64, 128, 256}.  Gate rows are contiguous when ldg = 0; otherwise the gate is read
 * in place from a wider tensor as lines of gpl rows (gpl * dim contiguous channels, e.g. the heads of one token)
 * ldg elements apart: row r at (r / gpl) * ldg + (r % gpl) * dim (rows a multiple of gpl, ldg * sizeof(dtype) a
 * multiple of 16, such as the gate columns of a fused input projection).  The backward writes dx, dgate (rows
 * contiguous) and dweight (if non-NULL; summed over rows in a fixed order through the workspace). */
int gdn_gated_rmsnorm_fwd(const void* x, const void* gate, int64_t ldg, int gpl, const float* weight, void* y,
                          int64_t rows, int dim, float eps, int dtype, void* stream);
int gdn_gated_rmsnorm_bwd_ws_bytes(int64_t rows, int dim, size_t* bytes);
int gdn_gated_rmsnorm_bwd(const void* x, const void* gate, int64_t ldg, int gpl, const float* weight,
                          const void* dy, void* dx, void* dgate, float* dweight, void* ws, size_t ws_bytes,
                          int64_t rows, int dim, float eps, int dtype, void* stream);

/* L2 normalisation with a scale over rows of `dim` channels (one head of q or k):
 *   y = scale * x / max(||x||, eps)
 * Replaces the per-head normalisation of q and k (archbench/layers/nsgdn.py:527-528: F.normalize(.) * DK^-1/2,
 * and fla's use_qk_l2norm_in_kernel) where it is not fused into the short convolution.  x, y, dy, dx [rows, dim]
 * in dtype; dim in {64, 128, 256}; no workspace (no parameters). */
int gdn_l2norm_fwd(const void* x, void* y, int64_t rows, int dim, float eps, float scale, int dtype, void* stream);
int gdn_l2norm_bwd(const void* x, const void* dy, void* dx, int64_t rows, int dim, float eps, float scale, int dtype,
                   void* stream);

/* Decay and write-strength gates from their projections, per token and head:
 *   g    = max(-exp(A_log[h]) * softplus(a + dt_bias[h]), g_min)      (natural-log decay; g_min = -inf: none)
 *   beta = beta_scale * sigmoid(b + b_bias[h])
 * Replaces nsgdn.py:531-533 (la = -softplus(ab[:H] + dt_bias) * exp(A_log), clamp_min(la_min), beta =
 * sigmoid(ab[H:] + b_bias)) and fla GatedDeltaNet's g / beta (beta_scale 2 for allow_neg_eigval).  a, b, da, db
 * [ntok] rows of H in dtype, the rows of a and b lda elements apart, of da and db ldd apart (0 = H, contiguous;
 * 2H reads a and b as the halves of one [ntok, 2H] projection, as the reference slices ab, and writes its gradient
 * in place); A_log, dt_bias, b_bias [H] fp32 (dt_bias, b_bias may be NULL = 0); g, beta, dg, dbeta
 * [ntok, H] fp32.  The backward writes da, db and, where non-NULL, dA_log, ddt_bias, db_bias (summed over tokens
 * in a fixed order through the workspace). */
int gdn_gates_fwd(const void* a, const void* b, int64_t lda, const float* A_log, const float* dt_bias,
                  const float* b_bias, float* g, float* beta, int64_t ntok, int H, float beta_scale, float g_min,
                  int dtype, void* stream);
int gdn_gates_bwd_ws_bytes(int64_t ntok, int H, size_t* bytes);
int gdn_gates_bwd(const void* a, const void* b, int64_t lda, const float* A_log, const float* dt_bias,
                  const float* b_bias, const float* dg, const float* dbeta, void* da, void* db, int64_t ldd,
                  float* dA_log, float* ddt_bias, float* db_bias, void* ws, size_t ws_bytes, int64_t ntok, int H,
                  float beta_scale, float g_min, int dtype, void* stream);

/* Cross-entropy forward and backward in one pass, in place on a chunk of logits [N, ld] (dtype; V classes,
 * V % 8 == 0, ld % 8 == 0, V <= 65536): loss[i] = logsumexp(x_i) - x_i,target[i] (0 where target == ignore_index,
 * NaN for a target outside [0, V)), lse[i] (if non-NULL), and x_i <- dloss * (softmax(x_i) - onehot(target_i))
 * (zeros for ignored rows), with dloss read from a device scalar (NULL = 1).  Replaces fla's cross_entropy_fwd +
 * cross_entropy_bwd(inplace_backward=True) on each chunk of archbench's fused linear cross-entropy
 * (archbench/fused_ce.py:33-45); the chunk GEMMs around it stay library GEMMs. */
int gdn_cross_entropy_fwd_bwd(void* logits, const int64_t* target, float* loss, float* lse, const float* dloss,
                              int64_t N, int V, int64_t ld, int64_t ignore_index, int dtype, void* stream);

/* Write direction of the n-step family: per token row of K channels (one head of one token), with p the previous
 * token's key in the same sequence (zero at t = 0),
 *   u_1 = beta k,  u_{i+1} = u_i - lam beta (p . u_i) (p - (p . k) k)   for i < n_steps.
 * Replaces write_direction (archbench/layers/nsgdn.py:61-75) and the shift of k that feeds it (:535-536).  k, u, du,
 * dk [B, T, H, K] in dtype; beta, dbeta, dlam [B, T, H] fp32; lam [H] fp32 (the module's softplus(lam)).  The
 * backward writes dk (through both k and the next token's p), dbeta and dlam per row (the caller sums dlam over
 * B and T).  K in {64, 128, 256}, n_steps >= 1; fp32 arithmetic. */
int gdn_write_direction_fwd(const void* k, const float* beta, const float* lam, void* u, int B, int T, int H, int K,
                            int n_steps, int dtype, void* stream);
int gdn_write_direction_bwd(const void* k, const float* beta, const float* lam, const void* du, void* dk,
                            float* dbeta, float* dlam, int B, int T, int H, int K, int n_steps, int dtype,
                            void* stream);

/* Exact fp32 token scan of the n-step family: the reference's "triton" / "ref" scan, archbench::nsgdn_fwd and
 * archbench::nsgdn_bwd (archbench/layers/nsgdn.py:80-154, ops :162-216, the recurrence of nsgdn_ref :408-417).
 * Per token, with the state S [V, K] from zero: S <- e^{la} S, r = v - S k, S <- S + r u^T, y = S q.  q, k, u
 * [B, T, H, K], v, y, r [B, T, H, V], la [B, T, H], all fp32 (q already scaled, as the reference's module does).
 * The forward writes y, the residuals r and the state every ct tokens into st (the backward's checkpoints); the
 * backward writes dv directly and dq, du, dk, dla as n_partials row blocks each ([n_partials][B*T*H][K],
 * [n_partials][B*T*H]) that the caller sums over the first index (the reference adds them with atomics).  Sizes
 * of st, of the backward's scratch and n_partials from gdn_token_scan_sizes.  K in {64, 128}, any V.
 * Optional states, an extension of the reference's zero-initialised scan (NULL: none), in fla's [B, H, K, V] fp32
 * layout: h0 (initial) and hT (final) in the forward, dhT and dh0 in the backward; B * T == 0 returns at once
 * without touching them. */
int gdn_token_scan_sizes(int B, int T, int H, int K, int V, size_t* st_bytes, size_t* scratch_bytes,
                         int* n_partials);
int gdn_token_scan_fwd(const float* q, const float* k, const float* u, const float* v, const float* la,
                       const float* h0, float* y, float* r, float* st, size_t st_bytes, float* hT, int B, int T, int H,
                       int K, int V, void* stream);
int gdn_token_scan_bwd(const float* q, const float* k, const float* u, const float* la, const float* r,
                       const float* st, size_t st_bytes, const float* dy, const float* dhT, float* dv, float* dq_part,
                       float* du_part, float* dk_part, float* dla_part, float* dh0, float* scratch,
                       size_t scratch_bytes, int B, int T, int H, int K, int V, void* stream);

/* Per-stage kernel timing (diagnostic; no counterpart in the reference, which times whole phases with CUDA
 * events in archbench/logger.py:57-81).  While enabled (process-wide: launches from any host thread count), every
 * kernel the calls above enqueue is bracketed by hipEvents on the same stream.  gdn_profile_read synchronises on those events and
 * returns, per stage, the summed milliseconds and the number of launches (arrays of at least
 * GDN_PROFILE_STAGES entries), then clears the record.  Stage names: gdn_profile_stage_name. */
#define GDN_PROFILE_STAGES 23
int gdn_profile_enable(int on);
int gdn_profile_read(double* ms_sum, int* launches, int n_stages);
const char* gdn_profile_stage_name(int stage);

#ifdef __cplusplus
}
#endif

#endif /* GDN_MI355X_H */
