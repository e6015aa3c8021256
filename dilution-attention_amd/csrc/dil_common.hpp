// Shared device helpers for the gfx950 dilution-attention kernels.
//
// Conventions used by every kernel in this library:
//   * Tensors on the path are row-major (rows, D) per (batch*head) slice with
//     64-bit slice strides passed explicitly.  D is a template parameter in
//     {16, 32, 64, 128}, and 256 for bf16 operands and the decode step.
//   * Matrix products use the 32x32 MFMA family: bf16 operands
//     (v_mfma_f32_32x32x16_bf16), fp32 operands (v_mfma_f32_32x32x2_f32), or
//     split operands (fp32 values as bf16 hi + lo pairs, three bf16 MFMAs per
//     step: the "tf32" precision); all accumulate in fp32 and share one
//     accumulator layout:
//       lane l, register i  ->  column (l & 31), row 8*(i>>2) + 4*(l>>5) + (i&3).
//   * An operand tile of 32 rows x K is held one row per lane (row = l & 31);
//     the two lane halves (h = l >> 5) hold two disjoint halves of the K index
//     set.  Which K indices a lane half holds is free as long as both operands
//     of a product use the same assignment; the helpers below fix one.
//   * Row permutation rho (swap bits 2 and 3 of the row index within a
//     32-row tile).  Loading an A operand with lane l holding logical row
//     rho(l & 31) makes accumulator register i of lane half h hold logical
//     row R(i, h) = 16*(i>>3) + 8*h + (i&7): two runs of 8 consecutive rows.
//     That layout is directly the B (or A) operand of a following product
//     whose contraction runs over those rows, with k slots 16*s + 8*h + t.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace dil {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr float kEps = 1e-9f;                    // reference kernels.py:66-67
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Storage dtypes understood by the C ABI (include/dilution_hip.h).
enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

// ---------------------------------------------------------------------------
// scalar conversions

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Load 8 consecutive elements of storage dtype `dt` as fp32.
__device__ __forceinline__ void load8_f32(const void* base, int64_t idx, int dt, float (&o)[8]) {
  if (dt == DT_F32) {
    const floatx4* p = reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + idx);
    floatx4 a = p[0], b = p[1];
    o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
    o[4] = b[0]; o[5] = b[1]; o[6] = b[2]; o[7] = b[3];
  } else {
    u16x8 r = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(base) + idx);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = (dt == DT_BF16) ? bf16_bits_to_f32(r[e]) : f16_bits_to_f32(r[e]);
  }
}

__device__ __forceinline__ void store_as(void* base, int64_t idx, int dt, float v) {
  if (dt == DT_F32) static_cast<float*>(base)[idx] = v;
  else if (dt == DT_BF16) static_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(v);
  else static_cast<uint16_t*>(base)[idx] = f32_to_f16_bits(v);
}

// Store 4 fp32 values as 4 consecutive elements of storage dtype `dt` (the
// rounding of store_as) in one store: idx is a multiple of 4.
__device__ __forceinline__ void store4_as(void* base, int64_t idx, int dt, const floatx4& v) {
  if (dt == DT_F32) {
    *reinterpret_cast<floatx4*>(static_cast<float*>(base) + idx) = v;
  } else {
    u16x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (dt == DT_BF16) ? f32_to_bf16_bits(v[e]) : f32_to_f16_bits(v[e]);
    *reinterpret_cast<u16x4*>(static_cast<uint16_t*>(base) + idx) = r;
  }
}

// Store 8 fp32 values as 8 consecutive elements of storage dtype `dt` (the
// rounding of store_as), in 16-byte stores: idx is a multiple of 8 and the
// base 16-byte aligned.
__device__ __forceinline__ void store8_as(void* base, int64_t idx, int dt, const float (&v)[8]) {
  if (dt == DT_F32) {
    floatx4* p = reinterpret_cast<floatx4*>(static_cast<float*>(base) + idx);
    p[0] = floatx4{v[0], v[1], v[2], v[3]};
    p[1] = floatx4{v[4], v[5], v[6], v[7]};
  } else {
    u16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (dt == DT_BF16) ? f32_to_bf16_bits(v[e]) : f32_to_f16_bits(v[e]);
    *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(base) + idx) = r;
  }
}

// ---------------------------------------------------------------------------
// MFMA traits: compute type CT is __bf16, float or split32.

// Storage element of split operands: an fp32 value x held as hi = bf16(x)
// and lo = bf16(x - hi), both rounded to nearest even, so hi + lo is x to
// within 2^-17 |x|.  Eight consecutive elements are stored as their eight hi
// halves, then their eight lo halves (32 bytes); every access of a split
// tile touches whole groups of eight that start at a multiple of 8 elements.
struct split32 {
  uint32_t bits;
};
struct SplitFrag {
  bf16x8 hi, lo;
};

template <typename CT> struct Mma;

template <> struct Mma<__bf16> {
  static constexpr int kPerLane = 8;      // K elements a lane contributes per instruction
  static constexpr int kStep = 16;        // K covered by one instruction
  using frag = bf16x8;
  __device__ static __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // b holds values exact in the operand type (identity, ones)
  __device__ static __forceinline__ floatx16 mma_bexact(frag a, frag b, floatx16 c) { return mma(a, b, c); }
  // Pack 8 fp32 values into one operand fragment (round to nearest even).
  __device__ static __forceinline__ frag pack(const float* v) {
    floatx2 p0 = {v[0], v[1]}, p1 = {v[2], v[3]}, p2 = {v[4], v[5]}, p3 = {v[6], v[7]};
    bf16x2 b0 = __builtin_convertvector(p0, bf16x2);
    bf16x2 b1 = __builtin_convertvector(p1, bf16x2);
    bf16x2 b2 = __builtin_convertvector(p2, bf16x2);
    bf16x2 b3 = __builtin_convertvector(p3, bf16x2);
    frag f = {b0[0], b0[1], b1[0], b1[1], b2[0], b2[1], b3[0], b3[1]};
    return f;
  }
};

template <> struct Mma<float> {
  static constexpr int kPerLane = 1;
  static constexpr int kStep = 2;
  using frag = float;
  __device__ static __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ floatx16 mma_bexact(frag a, frag b, floatx16 c) { return mma(a, b, c); }
  __device__ static __forceinline__ frag pack(const float* v) { return v[0]; }
};

// a b ~ a.hi b.hi + a.hi b.lo + a.lo b.hi: the dropped a.lo b.lo and the
// rounding of lo leave an error below 2^-15 |a||b| per product term, finer
// than the 10-bit mantissa of tf32 operands.
template <> struct Mma<split32> {
  static constexpr int kPerLane = 8;
  static constexpr int kStep = 16;
  using frag = SplitFrag;
  __device__ static __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.lo, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.lo, b.hi, c, 0, 0, 0);
  }
  // b exact in bf16 (its lo half is zero): two products
  __device__ static __forceinline__ floatx16 mma_bexact(frag a, frag b, floatx16 c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.hi, b.hi, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.lo, b.hi, c, 0, 0, 0);
  }
  __device__ static __forceinline__ frag pack(const float* v) {
    frag f;
    f.hi = Mma<__bf16>::pack(v);
    float r[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) r[t] = v[t] - static_cast<float>(f.hi[t]);
    f.lo = Mma<__bf16>::pack(r);
    return f;
  }
};

// Operand types whose fragments carry 8 K elements per lane (bf16 and split)
template <typename CT> constexpr bool kWideFrag = Mma<CT>::kPerLane == 8;

// The C ABI's precision code of an operand type (0 "ieee", 1 "tf32", 2
// "bf16"), and the storage dtype that already is the operand type (-1: none,
// split operands are always built)
template <typename CT>
constexpr int kOperandPrec = std::is_same_v<CT, __bf16> ? 2 : std::is_same_v<CT, split32> ? 1 : 0;
template <typename CT>
constexpr int kNativeDtype = std::is_same_v<CT, __bf16> ? DT_BF16 : std::is_same_v<CT, float> ? DT_F32 : -1;
inline int native_dtype(int prec) { return prec == 2 ? DT_BF16 : prec == 0 ? DT_F32 : -1; }

// The fragment of 8 consecutive K elements starting at p (a group start)
template <typename CT>
__device__ __forceinline__ typename Mma<CT>::frag frag8_at(const CT* p) {
  if constexpr (std::is_same_v<CT, split32>) {
    const bf16x8* q = reinterpret_cast<const bf16x8*>(p);
    return SplitFrag{q[0], q[1]};
  } else {
    return *reinterpret_cast<const bf16x8*>(p);
  }
}

// Row permutation within a 32-row tile: swap bits 2 and 3 (an involution).
__device__ __forceinline__ int rho(int m) {
  return (m & ~0xC) | ((m & 4) << 1) | ((m & 8) >> 1);
}
// Logical row held by accumulator register i of lane half h when the
// A operand was loaded rho-permuted.
__device__ __forceinline__ int perm_row(int i, int h) { return 16 * (i >> 3) + 8 * h + (i & 7); }
// Row held by accumulator register i of lane half h without permutation.
__device__ __forceinline__ int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// ---------------------------------------------------------------------------
// Operand tiles of 32 rows x D (contraction over D).
//
// Lane l holds row (l & 31), K indices [h*D/2, (h+1)*D/2) of it (h = l >> 5),
// converted to the compute type.  Instruction s uses the lane's K indices
// h*D/2 + s*kPerLane + [0, kPerLane).

template <typename CT, int D> struct RowFrag {
  static constexpr int kSteps = D / (2 * Mma<CT>::kPerLane);
  typename Mma<CT>::frag f[kSteps];
};

// Load one row segment (D/2 elements starting at `src`) of compute type CT
// from a buffer that already holds the compute type.
template <typename CT, int D>
__device__ __forceinline__ void load_row_frag(RowFrag<CT, D>& rf, const CT* src) {
  if constexpr (kWideFrag<CT>) {
#pragma unroll
    for (int s = 0; s < RowFrag<CT, D>::kSteps; ++s) rf.f[s] = frag8_at<CT>(src + 8 * s);
  } else {
    const floatx4* p = reinterpret_cast<const floatx4*>(src);
#pragma unroll
    for (int s = 0; s < RowFrag<CT, D>::kSteps / 4; ++s) {
      floatx4 x = p[s];
      rf.f[4 * s + 0] = x[0]; rf.f[4 * s + 1] = x[1];
      rf.f[4 * s + 2] = x[2]; rf.f[4 * s + 3] = x[3];
    }
    if constexpr (RowFrag<CT, D>::kSteps % 4 != 0) {
#pragma unroll
      for (int s = (RowFrag<CT, D>::kSteps / 4) * 4; s < RowFrag<CT, D>::kSteps; ++s) rf.f[s] = src[s];
    }
  }
}

template <typename CT, int D>
__device__ __forceinline__ void zero_row_frag(RowFrag<CT, D>& rf) {
#pragma unroll
  for (int s = 0; s < RowFrag<CT, D>::kSteps; ++s) rf.f[s] = typename Mma<CT>::frag{};
}

// acc += A(32 x D) * B(32 x D)^T for two row-fragment tiles.
template <typename CT, int D>
__device__ __forceinline__ floatx16 mma_rows(const RowFrag<CT, D>& a, const RowFrag<CT, D>& b, floatx16 acc) {
#pragma unroll
  for (int s = 0; s < RowFrag<CT, D>::kSteps; ++s) acc = Mma<CT>::mma(a.f[s], b.f[s], acc);
  return acc;
}

// The same with A's row segment read from memory (an LDS row tile) one
// instruction's fragment at a time, so that a wide A never sits in registers
// whole (head_dim 256; 8-element fragment types).
template <typename CT, int D>
__device__ __forceinline__ floatx16 mma_rows_src(const CT* a_src, const RowFrag<CT, D>& b, floatx16 acc) {
  static_assert(kWideFrag<CT>, "one 8-element fragment per instruction");
#pragma unroll
  for (int s = 0; s < RowFrag<CT, D>::kSteps; ++s) acc = Mma<CT>::mma(frag8_at<CT>(a_src + 8 * s), b.f[s], acc);
  return acc;
}

// ---------------------------------------------------------------------------
// wave-level helpers

__device__ __forceinline__ float partner32(float x) {   // value held by lane l ^ 32
  return __shfl_xor(x, 32, 64);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace dil
