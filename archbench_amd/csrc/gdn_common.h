// Shared device helpers for the gated DeltaNet kernels (gfx950 / CDNA4).
//
// Matrix products use the 16x16 MFMA output tile.  Operand fragments always hold 8 consecutive k values per
// lane: lane l covers outer index (l & 15) and k = 8*(l >> 4) + j, j = 0..7.  For bf16 one
// v_mfma_f32_16x16x32_bf16 consumes the fragment pair; for fp32 eight v_mfma_f32_16x16x4_f32 issue one k
// slice each (slice j takes k = 8*g + j from lane group g), which is the same sum over k in another order.
// The fp32 accumulator of a 16x16 tile holds rows 4*(l >> 4) + i (i = 0..3) of column (l & 15).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

constexpr int CH = 64;         // tokens per chunk
constexpr int NWAVE = 4;       // waves per workgroup
constexpr int NTHR = 64 * NWAVE;

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Word 3 of a raw buffer resource (__builtin_amdgcn_make_buffer_rsrc) on CDNA: 32-bit data format.  Buffer
// accesses take a uniform base in SGPRs and a 32-bit per-lane byte offset, and the hardware range check returns
// zeros for loads (and drops stores) at or past num_records.
constexpr int BUF_RSRC_WORD3 = 0x00020000;

template <typename T> struct Frag;
template <> struct Frag<bf16> { using type = bf16x8; };
template <> struct Frag<float> { using type = f32x8; };

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return static_cast<float>(x); }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return static_cast<bf16>(x); }
// a0 b0 + a1 b1 + c: for bf16 one v_dot2c_f32_bf16 (exact bf16 products, fp32 sum) in place of four conversions
// and two FMAs
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2(bf16 a0, bf16 a1, bf16 b0, bf16 b1, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(bf16x2{a0, a1}, bf16x2{b0, b1}, c, false);
}
__device__ __forceinline__ float dot2(float a0, float a1, float b0, float b1, float c) {
  return fmaf(a1, b1, fmaf(a0, b0, c));
}

__device__ __forceinline__ void mma(f32x4& c, const bf16x8& a, const bf16x8& b) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& c, const f32x8& a, const f32x8& b) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
}

// Lane-dependent helpers take the lane as a trailing argument (default: this thread's lane).  A kernel that
// loops over work items passes a lane value re-derived in every iteration, so that the address arithmetic is
// redone there rather than hoisted out of the loop and held in registers for its whole length.

// Fragment with k contiguous: element (o, k) at p[o * ld + k].
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_kc(const T* p, int ld, int o0, int k0, int l = lane_id()) {
  const T* s = p + (o0 + (l & 15)) * ld + k0 + 8 * (l >> 4);
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const bf16x8*>(s);
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(s);
    const f32x4 b = *reinterpret_cast<const f32x4*>(s + 4);
    return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
}

// Fragment with the outer index contiguous: element (o, k) at p[k * ld + o].
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_oc(const T* p, int ld, int o0, int k0, int l = lane_id()) {
  const T* s = p + (k0 + 8 * (l >> 4)) * ld + o0 + (l & 15);
  typename Frag<T>::type f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = s[j * ld];
  return f;
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_oct(const T* p, int ld, int o0, int k0, int l = lane_id());

template <bool KC, typename T>
__device__ __forceinline__ typename Frag<T>::type frag(const T* p, int ld, int o0, int k0, int l = lane_id()) {
  if constexpr (KC) return frag_kc(p, ld, o0, k0, l);
  else return frag_oct(p, ld, o0, k0, l);
}

// c += A[m0:m0+16, 0:KD] * B[0:KD, n0:n0+16].
//   A element (m, k): AKC ? A[m*lda + k] : A[k*lda + m]
//   B element (k, n): BKC ? B[n*ldb + k] : B[k*ldb + n]
template <bool AKC, bool BKC, int KD, typename T>
__device__ __forceinline__ void mma_blk(f32x4& c, const T* A, int lda, int m0, const T* B, int ldb, int n0,
                                        int l = lane_id()) {
#pragma unroll
  for (int k0 = 0; k0 < KD; k0 += 32) {
    const auto a = frag<AKC>(A, lda, m0, k0, l);
    const auto b = frag<BKC>(B, ldb, n0, k0, l);
    mma(c, a, b);
  }
}

// ---- permuted-k fragments ---------------------------------------------------------------------------------
// A pair of accumulator tiles covering rows [0,16) and [16,32) of a 32-row block holds, in lane group g,
// rows 4g..4g+3 of the first tile and 16+4g..16+4g+3 of the second.  Using those 8 rows as the k-slots of a
// fragment (slot p -> row 4g+p for p < 4, 16+4g+p-4 for p >= 4) lets an accumulator feed the next product as
// its B operand without leaving registers; the other operand is then read with the same slot order.
// k contiguous (element (o, k) at p[o*ld + k]), permuted slots: two 4-element reads.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_kc_perm(const T* p, int ld, int o0, int k0,
                                                              int l = lane_id()) {
  const T* s = p + (o0 + (l & 15)) * ld + k0 + 4 * (l >> 4);
  if constexpr (sizeof(T) == 2) {
    const bf16x4 a = *reinterpret_cast<const bf16x4*>(s);
    const bf16x4 b = *reinterpret_cast<const bf16x4*>(s + 16);
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(s);
    const f32x4 b = *reinterpret_cast<const f32x4*>(s + 16);
    return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
}

// outer index contiguous (element (o, k) at p[k*ld + o]), permuted slots.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_oc_perm(const T* p, int ld, int o0, int k0,
                                                              int l = lane_id()) {
  const T* s = p + (k0 + 4 * (l >> 4)) * ld + o0 + (l & 15);
  typename Frag<T>::type f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = s[j * ld];
    f[4 + j] = s[(16 + j) * ld];
  }
  return f;
}

// ---- transposing LDS reads (bf16) ---------------------------------------------------------------------------
// ds_read_b64_tr_b16: inside each 16-lane group, local lane m reads 4 bf16 at its address and lane i receives
// element (i mod 4) of the loads of lanes 4j + i/4, j = 0..3.  With local lane m pointing at row kb + m/4,
// columns o0 + 4(m mod 4) of a row-major tile, lane i receives the 4 values at rows kb..kb+3 of column o0 + i:
// a column-major operand slice read straight from a row-major tile.
typedef short shortx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x4 ld_tr4(const bf16* p, int ld, int o0, int kb, int l = lane_id()) {
  const int m = l & 15;
  const bf16* a = p + (kb + (m >> 2)) * ld + o0 + 4 * (m & 3);
  const shortx4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4*)(a));
  return __builtin_bit_cast(bf16x4, r);
}

// Fragment of an operand stored outer-contiguous (element (o, k) at p[k*ld + o]).
//   frag_oct:      plain slots (k = k0 + 8g + e)
//   frag_oct_perm: permuted slots (k = k0 + 4g + e, k0 + 16 + 4g + e)
// bf16 uses two transposing reads; fp32 falls back to scalar reads.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_oct(const T* p, int ld, int o0, int k0, int l) {
  if constexpr (sizeof(T) == 2) {
    const int g = l >> 4;
    const bf16x4 a = ld_tr4(p, ld, o0, k0 + 8 * g, l), b = ld_tr4(p, ld, o0, k0 + 8 * g + 4, l);
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
    return frag_oc(p, ld, o0, k0, l);
  }
}
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_oct_perm(const T* p, int ld, int o0, int k0,
                                                               int l = lane_id()) {
  if constexpr (sizeof(T) == 2) {
    const int g = l >> 4;
    const bf16x4 a = ld_tr4(p, ld, o0, k0 + 4 * g, l), b = ld_tr4(p, ld, o0, k0 + 16 + 4 * g, l);
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
    return frag_oc_perm(p, ld, o0, k0, l);
  }
}

// Fragment from two accumulator tiles (rows [0,16) and [16,32) of a 32-row block), permuted slots.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type frag_acc2(const f32x4& t0, const f32x4& t1) {
  typename Frag<T>::type f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = from_f<T>(t0[j]);
    f[4 + j] = from_f<T>(t1[j]);
  }
  return f;
}

__device__ __forceinline__ int acc_row(int i, int l = lane_id()) { return 4 * (l >> 4) + i; }
__device__ __forceinline__ int acc_col(int l = lane_id()) { return l & 15; }

// Workgroup -> (V block, head) for the chunk sweeps.  Workgroups are dispatched round-robin over the 8 XCDs
// (each with its own L2), so with a plain grid the NV V-block workgroups of one head land on different XCDs and
// each reads the head's q/k from HBM.  With a 1-D grid of NV * BH workgroups and BH a multiple of 8, linear id L
// runs on XCD L % 8; giving slot s = L / 8 of XCD x the head 8 * (s / NV) + x and V block s % NV keeps a head's
// V blocks on one XCD, dispatched back to back, so the second read of its q/k is an L2 hit.
__device__ __forceinline__ void sweep_block(int NV, int BH, int& vb, int& bh) {
  const int L = blockIdx.x;
  if ((BH & 7) == 0) {
    const int x = L & 7, s = L >> 3;
    bh = 8 * (s / NV) + x;
    vb = s - (s / NV) * NV;
  } else {
    bh = L / NV;
    vb = L - bh * NV;
  }
}

// Sum over the 16 lanes of a DPP row (the columns of one accumulator tile row set), left in every lane of the
// row: butterfly on DPP, no LDS crossbar.  quad_perm [1,0,3,2] and [2,3,0,1] sum each quad, row_half_mirror
// (lane i <- 7 - i) adds the other quad of the half-row, row_mirror (lane i <- 15 - i) the other half-row.
// Every DPP move here reads a lane of its own row, all of which are active, so bound_ctrl (zero for a source
// lane that is not there) changes no value; it lets the compiler fold the move into the add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_sum_step(float x) {
  return x + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float sum16(float x) {
  x = dpp_sum_step<0xb1>(x);   // quad_perm [1,0,3,2]
  x = dpp_sum_step<0x4e>(x);   // quad_perm [2,3,0,1]
  x = dpp_sum_step<0x141>(x);  // row_half_mirror
  x = dpp_sum_step<0x140>(x);  // row_mirror
  return x;
}

// hardware reciprocal (1 ulp) in place of an IEEE division, and the logistic function on it
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_sigmoid(float z) { return fast_rcp(1.f + __expf(-z)); }

// 8 consecutive elements of a row as loaded (16 B in bf16, 32 B in fp32), converted to fp32 at use.  The row
// kernels read and write each element once, so loads and stores carry the nontemporal hint (measured: the
// gated RMSNorm forward 77 -> 67 us, the cross-entropy kernel 634 -> 573 us)
template <typename T>
struct Row8;
template <>
struct Row8<bf16> {
  bf16x8 r;
  __device__ __forceinline__ void load(const bf16* p) { r = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p)); }
  __device__ __forceinline__ void get(float (&v)[8]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(r[j]);
  }
};
template <>
struct Row8<float> {
  f32x4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
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
__device__ __forceinline__ void store_row8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = static_cast<bf16>(v[j]);
    __builtin_nontemporal_store(r, reinterpret_cast<bf16x8*>(p));
  } else {
    __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, reinterpret_cast<f32x4*>(p + 4));
  }
}

// Across the 16-lane rows of a wave, without the LDS crossbar: v_permlane16_swap returns x's rows (0,0,2,2) and
// (1,1,3,3), v_permlane32_swap rows (0,1,0,1) and (2,3,2,3) (each lane keeps its position inside the row), so one
// swap and one add (or max) combine lanes l and l ^ 16, or l and l ^ 32.
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// lanes l and l ^ 8 inside a row (row_ror:8)
__device__ __forceinline__ float xor8_sum(float x) { return dpp_sum_step<0x128>(x); }

// Sum / max over the whole wave, the result in every lane
__device__ __forceinline__ float wave_sum64(float x) { return xor32_sum(xor16_sum(sum16(x))); }
template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float x) {
  return fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, true)));
}
__device__ __forceinline__ float wave_max64(float x) {
  x = dpp_max_step<0xb1>(x);
  x = dpp_max_step<0x4e>(x);
  x = dpp_max_step<0x141>(x);
  x = dpp_max_step<0x140>(x);
  return xor32_max(xor16_max(x));
}

// Sum over aligned runs of LANES lanes (1, 2, 4, ..., 64), the same value left in every lane of the run: DPP
// butterflies within 16 lanes (as sum16), row swaps across rows.
template <int LANES>
__device__ __forceinline__ float lane_group_sum(float s) {
  if constexpr (LANES >= 2) s = dpp_sum_step<0xb1>(s);
  if constexpr (LANES >= 4) s = dpp_sum_step<0x4e>(s);
  if constexpr (LANES >= 8) s = dpp_sum_step<0x141>(s);
  if constexpr (LANES >= 16) s = dpp_sum_step<0x140>(s);
  if constexpr (LANES >= 32) s = xor16_sum(s);
  if constexpr (LANES >= 64) s = xor32_sum(s);
  return s;
}

// Inclusive prefix sum over the 64 lanes of a wave, on DPP: shifts within each 16-lane row, then the row
// totals broadcast forward (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float x) {
  const int t = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, true);
  return x + __int_as_float(t);
}
__device__ __forceinline__ float wave_inclusive_scan(float x) {
  x = dpp_add<0x111, 0xf>(x);  // row_shr:1
  x = dpp_add<0x112, 0xf>(x);  // row_shr:2
  x = dpp_add<0x114, 0xf>(x);  // row_shr:4
  x = dpp_add<0x118, 0xf>(x);  // row_shr:8
  x = dpp_add<0x142, 0xa>(x);  // row_bcast:15
  x = dpp_add<0x143, 0xc>(x);  // row_bcast:31
  return x;
}

}  // namespace gdn
