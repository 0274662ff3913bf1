// MFMA fragments for the 16x16 output tiles used by every GEMM kernel here.
//
// A wave computes D(16x16) += A(16 x KSTEP) * B(KSTEP x 16).  Lane l supplies
// row (l & 15) of A and column (l & 15) of B, each as VEC consecutive
// reduction elements starting at (l >> 4) * VEC:
//   fp32  : VEC = 4, KSTEP = 16, four v_mfma_f32_16x16x4_f32 (one per vector element)
//   f16/bf16: VEC = 8, KSTEP = 32, one v_mfma_f32_16x16x32_{f16,bf16}
// The hardware's assignment of (lane group, element) to a reduction index is
// the same for A and B, so any fixed assignment of reduction indices to
// (l >> 4, element) gives the same sum; loading VEC consecutive elements per
// lane keeps every fragment a single 16-byte load.
// D layout: lane l holds D[(l >> 4) * 4 + r][l & 15] in accumulator element r.
#pragma once

#include <hip/hip_runtime.h>

namespace st {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

template <typename T>
struct Frag;

template <>
struct Frag<float> {
  using type = v4f;
  static constexpr int VEC = 4;
  static constexpr int KSTEP = 16;
};
template <>
struct Frag<_Float16> {
  using type = v8h;
  static constexpr int VEC = 8;
  static constexpr int KSTEP = 32;
};
template <>
struct Frag<__bf16> {
  using type = v8bf;
  static constexpr int VEC = 8;
  static constexpr int KSTEP = 32;
};

__device__ __forceinline__ v4f mfma(const v4f& a, const v4f& b, v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc, 0, 0, 0);
  return acc;
}
__device__ __forceinline__ v4f mfma(const v8h& a, const v8h& b, v4f acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma(const v8bf& a, const v8bf& b, v4f acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

typedef __bf16 v4bf __attribute__((ext_vector_type(4)));

// hi/lo bf16 split of fp32 values (the split-operand fp32 products:
// x = hi + lo + d, |d| <= 2^-18 |x|), hi = bf16(x) and lo = bf16(x - hi),
// both rounded to nearest even.  A pair is converted by one packed
// conversion; each hi comes back to fp32 exactly as a shift (low half) or a
// mask (high half) of the packed word, so a value costs three VALU operations
// (half a conversion, the shift or mask, the subtraction, half a conversion)
// instead of four with a second conversion of each hi.
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){a, b}, v2bf));
}
__device__ __forceinline__ void split_pair(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16(a, b);
  lo = pack_bf16(a - __builtin_bit_cast(float, hi << 16), b - __builtin_bit_cast(float, hi & 0xFFFF0000u));
}
__device__ __forceinline__ void split4(const v4f& x, v4bf& hi, v4bf& lo) {
  uint32_t h[2], l[2];
  split_pair(x[0], x[1], h[0], l[0]);
  split_pair(x[2], x[3], h[1], l[1]);
  hi = __builtin_bit_cast(v4bf, h);
  lo = __builtin_bit_cast(v4bf, l);
}
// 8 consecutive values: x0 gives elements 0..3, x1 elements 4..7
__device__ __forceinline__ void split8(const v4f& x0, const v4f& x1, v8bf& hi, v8bf& lo) {
  uint32_t h[4], l[4];
  split_pair(x0[0], x0[1], h[0], l[0]);
  split_pair(x0[2], x0[3], h[1], l[1]);
  split_pair(x1[0], x1[1], h[2], l[2]);
  split_pair(x1[2], x1[3], h[3], l[3]);
  hi = __builtin_bit_cast(v8bf, h);
  lo = __builtin_bit_cast(v8bf, l);
}

// The same split of 4 values with a conversion per element (four operations
// a value).  It measured faster than split4 in the fp32 ring gather's B stage
// (config 2 forward 140 -> 123 us), where the stage overlaps the previous
// offset's MFMAs.
__device__ __forceinline__ void split4_each(const v4f& x, v4bf& hi, v4bf& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (__bf16)x[e];
    lo[e] = (__bf16)(x[e] - (float)hi[e]);
  }
}
// a*b ~= al*bh + ah*bl + ah*bh, in that order (every kernel that must agree
// bitwise with another adds the three products in this order)
__device__ __forceinline__ v4f mfma_x3(const v8bf& ah, const v8bf& al, const v8bf& bh, const v8bf& bl, v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::type zero_frag() {
  typename Frag<T>::type f;
#pragma unroll
  for (int e = 0; e < Frag<T>::VEC; ++e) f[e] = (T)0.0f;
  return f;
}

// Load VEC elements row[col .. col+VEC) with zero fill past `limit`.
// `vec_ok` promises row + col is 16-byte aligned whenever col + VEC <= limit.
template <typename T>
__device__ __forceinline__ typename Frag<T>::type load_frag(const T* __restrict__ row, int col, int limit,
                                                            bool vec_ok) {
  using F = typename Frag<T>::type;
  constexpr int VEC = Frag<T>::VEC;
  if (vec_ok && col + VEC <= limit) return *reinterpret_cast<const F*>(row + col);
  F f;
#pragma unroll
  for (int e = 0; e < VEC; ++e) f[e] = (col + e < limit) ? row[col + e] : (T)0.0f;
  return f;
}

// Raw buffer resource over [base, base + bytes), bytes < 2^31 (gfx9-family
// descriptor, word 3 = 32-bit data format).  A 16-byte load at a byte offset
// past the end returns zeros and touches no memory: kOobOffset marks a
// missing row without a clamp or a select.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
constexpr int kOobOffset = 0x7FFFFFF0;
template <typename V>
__device__ __forceinline__ V load16(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  static_assert(sizeof(V) == 16, "16-byte fragment");
  return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0));
}

template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return (T)v;
}

// Store epilogue of the gather-GEMMs, on the fp32 accumulator of (row r, column c):
//   v = (acc + bias[c]) * scale[c] + shift[c] + residual[r, c], then ReLU when relu is set
// bias (the convolution's, conv.py:227-228) and residual (n_dst x Nd, rows in
// output order: a residual block's shortcut, blocks.py:121-124) have the
// output dtype; scale and shift are fp32 (an evaluation-mode batch norm folded
// to one affine map per channel, nn/functional/norm.py:105-112).  A null
// pointer drops its term.
template <typename T>
struct Epi {
  static constexpr bool kReads = true;  // reads memory per element (the residual)
  const T* bias;
  const float* scale;
  const float* shift;
  const T* residual;
  int relu;
  __device__ __forceinline__ void column(int col, int Nd, float& mul, float& add) const {
    const float b = (bias && col < Nd) ? (float)bias[col] : 0.f;
    if (scale && col < Nd) {
      mul = scale[col];
      add = b * mul + (shift ? shift[col] : 0.f);
    } else {
      mul = 1.f;
      add = b;
    }
  }
  __device__ __forceinline__ float apply(float acc, float mul, float add, int64_t row, int Nd, int col) const {
    float v = scale ? fmaf(acc, mul, add) : acc + add;
    if (residual) v += (float)residual[row * Nd + col];
    return (relu && v < 0.f) ? 0.f : v;  // (a NaN stays NaN, as under torch.relu)
  }
};
// The store epilogue of the plain convolution: acc + bias[c] and nothing
// else, so the store loop has no other memory access (the general epilogue's
// possible residual read, which may alias the output, serialises the stores:
// the split-fp32 gather measured 152 vs 184 us).
template <typename T>
struct BiasEpi {
  static constexpr bool kReads = false;
  const T* bias;
  __device__ __forceinline__ void column(int col, int Nd, float& mul, float& add) const {
    mul = 1.f;
    add = (bias && col < Nd) ? (float)bias[col] : 0.f;
  }
  __device__ __forceinline__ float apply(float acc, float, float add, int64_t, int, int) const { return acc + add; }
};

template <typename T>
inline Epi<T> bias_epi(const void* bias) {
  return Epi<T>{(const T*)bias, nullptr, nullptr, nullptr, 0};
}

}  // namespace st
