// Device helpers shared by the DGDA prefill kernels (chunked MFMA path and the
// per-channel sub-chunk path): MFMA wrappers, bf16 hi/lo splitting, LDS operand reads,
// wave scans, the segment map S <- M S + N and the slot geometry of the sequence-
// parallel passes.
#pragma once
#include "maba_common.h"
#include <type_traits>

namespace maba {

typedef __attribute__((ext_vector_type(8))) short i16x8;

constexpr int PITCH = 72;     // bf16 row pitch of 64-wide LDS matrices (144 B: 16-B aligned, conflict-light)

// ------------------------------------------------------------------ MFMA helpers

__device__ __forceinline__ f32x4 mma32(f32x4 c, i16x8 a, i16x8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mma16(f32x4 c, i16x4 a, i16x4 b) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ short bf16_rn(float f) { return __builtin_bit_cast(short, (__bf16)f); }
__device__ __forceinline__ float bf16_val(short h) { return bf16_bits_to_f32((uint16_t)h); }

// Split four fp32 values into bf16 hi and lo parts (x ~= hi + lo), using the
// hardware round-to-nearest-even conversion (v_cvt_pk_bf16_f32).
// Two fp32 values to packed bf16 (round to nearest even), the first in the low half:
// one v_cvt_pk_bf16_f32.  Converting pairs (not 4-vectors) keeps the compiler on the
// packed form instead of re-deriving it from single conversions and byte permutes.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  typedef __attribute__((ext_vector_type(2))) float f32x2;
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// x - hi for the element of a packed bf16 pair selected by SEL (0: low half), as one
// v_dot2c_f32_bf16: (hi0, hi1) . (-1, -0) + x (or (-0, -1)).  The products are exact and
// x - hi is representable in fp32, so the result is the exact remainder.  The unused
// half is -0, not +0: the compiler encodes the pair (-1, +0) as the inline constant
// -1.0, which the instruction reads as the 32-bit pattern (+0, -1) -- the wrong half --
// while (-1, -0) and (-0, -1) stay literals (checked bit for bit against x - float(hi)
// on 2^19 pairs of the gfx950 build).
template <int SEL>
__device__ __forceinline__ float bf16_rem(uint32_t hpair, float x) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  const bf16x2 neg1 = __builtin_bit_cast(bf16x2, SEL ? 0xbf808000u : 0x8000bf80u);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, hpair), neg1, x, false);
}

__device__ __forceinline__ void split4(f32x4 x, i16x4& hi, i16x4& lo) {
  typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
  const uint32_t h01 = cvt_pk_bf16(x[0], x[1]), h23 = cvt_pk_bf16(x[2], x[3]);
  const f32x4 r = {bf16_rem<0>(h01, x[0]), bf16_rem<1>(h01, x[1]), bf16_rem<0>(h23, x[2]), bf16_rem<1>(h23, x[3])};
  const u32x2 hv = {h01, h23}, lv = {cvt_pk_bf16(r[0], r[1]), cvt_pk_bf16(r[2], r[3])};
  hi = __builtin_bit_cast(i16x4, hv);
  lo = __builtin_bit_cast(i16x4, lv);
}

// Four fp32 values to bf16, packed.
__device__ __forceinline__ bf16x4 to_bf16x4(f32x4 x) {
  typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
  const u32x2 v = {cvt_pk_bf16(x[0], x[1]), cvt_pk_bf16(x[2], x[3])};
  return __builtin_bit_cast(bf16x4, v);
}

__device__ __forceinline__ i16x8 cat8(i16x4 a, i16x4 b) {
  i16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

__device__ __forceinline__ i16x4 lds4(const short* base, int row, int col, int pitch) {
  return *(const i16x4*)(base + row * pitch + col);
}
__device__ __forceinline__ i16x8 lds8(const short* base, int row, int col, int pitch) {
  return *(const i16x8*)(base + row * pitch + col);
}
// Permuted-K A operand: columns c0..c0+3 and c0+16..c0+19 of one row.
__device__ __forceinline__ i16x8 lds4x2(const short* base, int row, int c0, int pitch) {
  return cat8(lds4(base, row, c0, pitch), lds4(base, row, c0 + 16, pitch));
}

// Transposed operand read (ds_read_b64_tr_b16).  Within each 16-lane group the
// instruction returns to lane i the elements src[4r + i/4][i%4] (r = 0..3), where
// src[j] are the four bf16 at lane j's address.  Addressing lane j of group g at
// row r0 + 4g + j/4, column c0 + 4(j%4) of a row-major matrix M therefore gives
// lane (c16, g) the column fragment M[r0 + 4g + r][c0 + c16], r = 0..3 -- the
// A (or B) operand fragment of M^T for a K-slice of 4 rows.
__device__ __forceinline__ i16x4 ldsT4(const short* base, int r0, int c0, int c16, int g, int pitch) {
  const short* p = base + (r0 + 4 * g + (c16 >> 2)) * pitch + c0 + 4 * (c16 & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p);
}
// Permuted-K operand of M^T: rows r0 + 4g..+3 and r0 + 16 + 4g..+3 of column c0 + c16.
__device__ __forceinline__ i16x8 ldsT4x2(const short* base, int r0, int c0, int c16, int g) {
  return cat8(ldsT4(base, r0, c0, c16, g, PITCH), ldsT4(base, r0 + 16, c0, c16, g, PITCH));
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves: shifts by 1, 2, 4, 8
// within each 16-lane row, then the row broadcasts of lanes 15 and 31.
__device__ __forceinline__ float wave_incl_scan(float x) {
  auto dpp = [](float v, auto ctrl_c, auto rmask_c, auto bound_c) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl_c)::value,
                                                      decltype(rmask_c)::value, 0xf, decltype(bound_c)::value));
  };
  using std::integral_constant;
  x += dpp(x, integral_constant<int, 0x111>{}, integral_constant<int, 0xf>{}, std::true_type{});  // row_shr:1
  x += dpp(x, integral_constant<int, 0x112>{}, integral_constant<int, 0xf>{}, std::true_type{});  // row_shr:2
  x += dpp(x, integral_constant<int, 0x114>{}, integral_constant<int, 0xf>{}, std::true_type{});  // row_shr:4
  x += dpp(x, integral_constant<int, 0x118>{}, integral_constant<int, 0xf>{}, std::true_type{});  // row_shr:8
  x += dpp(x, integral_constant<int, 0x142>{}, integral_constant<int, 0xa>{}, std::false_type{}); // row_bcast:15
  x += dpp(x, integral_constant<int, 0x143>{}, integral_constant<int, 0xc>{}, std::false_type{}); // row_bcast:31
  return x;
}

// LDS-only barrier: waits for this wave's LDS operations, not for its outstanding
// global loads (the next chunk's prefetch stays in flight across it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// S <- M S + N for a segment map X = [N | M] (64 x 128 fp32, row-major) on the slab
// Sr[kt][i] = S[16kt + 4g + i][col0 + c16] of one wave, with fp32 accuracy (M and S
// both split into bf16 hi/lo, three products).
__device__ __forceinline__ void apply_segment_map(const float* X, f32x4 (&Sr)[4], int col0, int c16, int g) {
  i16x4 Sh[4], Sl[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) split4(Sr[kt], Sh[kt], Sl[kt]);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    f32x4 acc;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = X[(16 * mt + 4 * g + i) * 128 + col0 + c16];  // N
    const int row = 16 * mt + c16;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // A operand: M[row][32p + 4g..+3] and [32p + 16 + 4g..+3]  (M lives in columns 64..127)
      const f32x4 m0 = *(const f32x4*)(X + row * 128 + 64 + 32 * p + 4 * g);
      const f32x4 m1 = *(const f32x4*)(X + row * 128 + 64 + 32 * p + 16 + 4 * g);
      i16x4 h0, l0, h1, l1;
      split4(m0, h0, l0);
      split4(m1, h1, l1);
      const i16x8 ah = cat8(h0, h1), al = cat8(l0, l1);
      const i16x8 bh8 = cat8(Sh[2 * p], Sh[2 * p + 1]), bl8 = cat8(Sl[2 * p], Sl[2 * p + 1]);
      acc = mma32(acc, ah, bh8);
      acc = mma32(acc, ah, bl8);
      acc = mma32(acc, al, bh8);
    }
    Sr[mt] = acc;
  }
}

// Segments of sequence bh (nchunks chunks) in slots of U chunks over the (b,h)-major
// order: the pieces of [bh * nchunks, (bh + 1) * nchunks) between multiples of U.
__device__ __forceinline__ int seg_count_of(int nchunks, int64_t U, int bh) {
  const int64_t s = (int64_t)bh * nchunks;
  return (int)((s + nchunks - 1) / U - s / U + 1);
}
__device__ __forceinline__ void seg_range_of(int nchunks, int64_t U, int bh, int k, int n, int& c0, int& c1) {
  const int64_t s = (int64_t)bh * nchunks, f = s / U;
  c0 = k == 0 ? 0 : (int)(U * (f + k) - s);
  c1 = k == n - 1 ? nchunks : (int)(U * (f + k + 1) - s);
}

// Slot geometry: U chunks per slot, at most nseg_max segments per sequence (1 when
// every sequence fits one slot: then slots are aligned to sequences).  Two output
// workgroups per CU, at least min_u chunks per slot.
struct SlotGeom { int64_t U; int nseg_max; };

inline SlotGeom slot_geom(int64_t BH, int64_t nch, int64_t min_u) {
  const int64_t slots = 2 * (int64_t)device_cu_count();
  int64_t U = (BH * nch + slots - 1) / slots;
  if (U < min_u) U = min_u;
  SlotGeom gm;
  if (nch <= U) {
    gm.U = nch;
    gm.nseg_max = 1;
  } else {
    gm.U = U;
    gm.nseg_max = (int)((nch - 1 + U - 1) / U + 1);
  }
  return gm;
}

// ------------------------------------------------------------------ layer prologue math

// The DGDA layer's activations (reference layers/dgda.py:103-121, 193-197) on the hardware
// transcendentals (a few ulp in fp32; outputs are then rounded to their dtype).
__device__ __forceinline__ float pro_sigmoid(float x) { return fast_rcp(1.f + fast_exp(-x)); }
__device__ __forceinline__ float pro_silu(float x) { return x * pro_sigmoid(x); }
// max(-softplus(x), -14) with torch's softplus (x itself above 20, where the clamp applies anyway);
// log(1 + e^x) loses e^x below fp32's epsilon, an absolute error under 1.2e-7
__device__ __forceinline__ float pro_log_decay(float x) {
  const float sp = x > 20.f ? x : fast_log(1.f + fast_exp(x));
  return fmaxf(-sp, -14.f);
}
// 1 / (||k|| + eps) from the sum of squares
__device__ __forceinline__ float pro_knorm_inv(float ss, float eps) { return fast_rcp(fast_sqrt(ss) + eps); }

// The conv history a fused layer prefill leaves (the inputs of its last three tokens per
// stream and channel); defined with the prologue kernels.
int launch_dgda_new_history(const maba_tensor* const* xs, const maba_tensor* const* hist,
                            maba_tensor* const* new_hist, hipStream_t stream);

}  // namespace maba
