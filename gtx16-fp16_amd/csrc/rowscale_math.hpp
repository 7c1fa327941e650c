// Row-rescale arithmetic shared by the rowscale cast kernel (rowscale.hip) and the GEMM kernels
// that cast their own activations (hgemm.hip): one definition, so both produce the same bits.
//
// Semantics (reference: src/gtx16_fp16/kernels.py:227-250):
//   amax_i = max_k |x[i,k]|, starting from 0, NaN ignored;
//   e_i    = ceil(log2(amax_i / thresh)) if amax_i > thresh else 0;
//   S_i    = 2^e_i;  y[i,k] = fp16_rne(x[i,k] * 2^-e_i).
// The exponent is computed from the fp32 bit fields (no log2/exp2): with thresh = 2^t and
// amax = 1.m * 2^E (normal, since amax > thresh), amax/thresh = 1.m * 2^(E-t), whose ceil(log2)
// is E - t when the mantissa field is zero and E - t + 1 otherwise. A row with amax = +inf gets
// S = +inf and y = x * 0.
#pragma once

#include "g16_common.hpp"

namespace g16 {

__device__ inline float chunk_absmax(float m, u32x4 v, float) {
  m = fmaxf(m, fabsf(__uint_as_float(v.x)));
  m = fmaxf(m, fabsf(__uint_as_float(v.y)));
  m = fmaxf(m, fabsf(__uint_as_float(v.z)));
  m = fmaxf(m, fabsf(__uint_as_float(v.w)));
  return m;
}

__device__ inline float lo_h(uint32_t d) { return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d & 0xffffu))); }
__device__ inline float hi_h(uint32_t d) { return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d >> 16))); }

__device__ inline float chunk_absmax(float m, u32x4 v, _Float16) {
  m = fmaxf(m, fabsf(lo_h(v.x)));
  m = fmaxf(m, fabsf(hi_h(v.x)));
  m = fmaxf(m, fabsf(lo_h(v.y)));
  m = fmaxf(m, fabsf(hi_h(v.y)));
  m = fmaxf(m, fabsf(lo_h(v.z)));
  m = fmaxf(m, fabsf(hi_h(v.z)));
  m = fmaxf(m, fabsf(lo_h(v.w)));
  m = fmaxf(m, fabsf(hi_h(v.w)));
  return m;
}

__device__ inline uint32_t pack2(float a, float b) {
  const uint16_t lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(a));
  const uint16_t hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(b));
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

// x * 2^-e: exact (ldexp keeps the sign of zero and never rounds a product here, since any
// fp32 result below the normal range is far below half the smallest fp16 subnormal). A row whose
// scale is +inf (e == kInfExp) maps to x * 0 like the reference's multiply by 1/inf. (A plain
// multiply by 2^-e is not used: the compiler fuses it with the fp16 conversion into an FMA with a
// +0 addend, which turns -0 into +0.)
constexpr int kInfExp = 1 << 20;
__device__ inline float scale_down(float x, int e) { return e == kInfExp ? x * 0.f : ldexpf(x, -e); }

// fp32 chunk: 4 values -> 4 fp16 (8 bytes).
__device__ inline u32x2 cast_scaled(u32x4 v, int e, float) {
  u32x2 o;
  o.x = pack2(scale_down(__uint_as_float(v.x), e), scale_down(__uint_as_float(v.y), e));
  o.y = pack2(scale_down(__uint_as_float(v.z), e), scale_down(__uint_as_float(v.w), e));
  return o;
}

// fp16 chunk: 8 values -> 8 fp16 (16 bytes).
__device__ inline u32x4 cast_scaled(u32x4 v, int e, _Float16) {
  u32x4 o;
  o.x = pack2(scale_down(lo_h(v.x), e), scale_down(hi_h(v.x), e));
  o.y = pack2(scale_down(lo_h(v.y), e), scale_down(hi_h(v.y), e));
  o.z = pack2(scale_down(lo_h(v.z), e), scale_down(hi_h(v.z), e));
  o.w = pack2(scale_down(lo_h(v.w), e), scale_down(hi_h(v.w), e));
  return o;
}

// Exponent e and scale S of a row with |max| amax (already reduced over the row, NaN dropped);
// texp = log2(thresh).
__device__ inline void row_exponent(float amax, int texp, int& e, float& sc) {
  e = 0;
  sc = 1.f;
  const uint32_t ab = __float_as_uint(amax);
  const int E = static_cast<int>((ab >> 23) & 0xffu) - 127;
  const bool gt = amax > __uint_as_float(static_cast<uint32_t>(texp + 127) << 23);
  if (gt) {
    if ((ab & 0x7f800000u) == 0x7f800000u) {  // +inf (NaN never reaches here: fmaxf drops it)
      sc = __uint_as_float(0x7f800000u);
      e = kInfExp;
    } else {
      e = E - texp + ((ab & 0x007fffffu) != 0u ? 1 : 0);
      sc = e + 127 >= 255 ? __uint_as_float(0x7f800000u) : __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
    }
  }
}

// thresh must be a positive, normal power of two; returns its exponent, or -1000 for any other
// value (the entry points reject it).
inline int thresh_exponent(float thresh) {
  uint32_t b;
  __builtin_memcpy(&b, &thresh, sizeof(b));
  const uint32_t ex = (b >> 23) & 0xffu;
  if ((b >> 31) != 0u || ex == 0u || ex == 0xffu || (b & 0x007fffffu) != 0u) return -1000;
  return static_cast<int>(ex) - 127;
}

}  // namespace g16
