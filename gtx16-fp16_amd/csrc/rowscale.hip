// Row rescale + fp16 cast for the quantised GEMM path (M > 8).
//
// Semantics (reference: src/gtx16_fp16/kernels.py:227-250, called from ops.py:86-90):
//   amax_i = max_k |x[i,k]|, starting from 0, NaN ignored;
//   e_i    = ceil(log2(amax_i / thresh)) if amax_i > thresh else 0;
//   S_i    = 2^e_i;  y[i,k] = fp16_rne(x[i,k] * 2^-e_i).
// The exponent is computed from the fp32 bit fields (no log2/exp2): with thresh = 2^t and
// amax = 1.m * 2^E (normal, since amax > thresh), amax/thresh = 1.m * 2^(E-t), whose ceil(log2)
// is E - t when the mantissa field is zero and E - t + 1 otherwise. A row with amax = +inf gets
// S = +inf and y = x * 0.
//
// Layout: one 64-lane wavefront per row, 4 rows per 256-thread workgroup. Each lane keeps up to
// CH 16-byte chunks of its row in registers, so the row is read from HBM once: max-reduce across
// the wavefront (no LDS, no barrier), then scale, convert and store from the registers. Rows longer
// than 64*CH chunks stream the remainder twice (the second read hits L2).
//
// Output layouts: row-major y[M,K], or the tile-packed layout the 256x256 GEMM streams (see
// packed_offset in g16_common.hpp): every 256-row x 32-column block of y is one contiguous 16 KB
// run, already in the order (and LDS swizzle) the GEMM's DMA writes into LDS, so that DMA reads
// whole 1 KB runs instead of 64-byte pieces of 256 different rows.
#include "g16_common.hpp"

namespace g16 {
namespace {

constexpr int kRowsPerBlock = 4;

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
__device__ inline void store_scaled(_Float16* y, u32x4 v, int e, float) {
  u32x2 o;
  o.x = pack2(scale_down(__uint_as_float(v.x), e), scale_down(__uint_as_float(v.y), e));
  o.y = pack2(scale_down(__uint_as_float(v.z), e), scale_down(__uint_as_float(v.w), e));
  *reinterpret_cast<u32x2*>(y) = o;
}

// fp16 chunk: 8 values -> 8 fp16 (16 bytes).
__device__ inline void store_scaled(_Float16* y, u32x4 v, int e, _Float16) {
  u32x4 o;
  o.x = pack2(scale_down(lo_h(v.x), e), scale_down(hi_h(v.x), e));
  o.y = pack2(scale_down(lo_h(v.y), e), scale_down(hi_h(v.y), e));
  o.z = pack2(scale_down(lo_h(v.z), e), scale_down(hi_h(v.z), e));
  o.w = pack2(scale_down(lo_h(v.w), e), scale_down(hi_h(v.w), e));
  *reinterpret_cast<u32x4*>(y) = o;
}

// Where input chunk idx of `row` goes: row-major, or tile-packed (an fp32 input chunk is half of
// a 16-byte fp16 output chunk).
template <typename TX, bool PACK>
__device__ inline _Float16* out_at(_Float16* Y, int row, int K, int idx, int nks) {
  constexpr int EPC = 16 / static_cast<int>(sizeof(TX));
  if constexpr (!PACK) {
    return Y + static_cast<size_t>(row) * K + static_cast<size_t>(idx) * EPC;
  } else if constexpr (EPC == 8) {
    return reinterpret_cast<_Float16*>(reinterpret_cast<unsigned char*>(Y) + packed_offset(row, idx, nks));
  } else {
    return reinterpret_cast<_Float16*>(reinterpret_cast<unsigned char*>(Y) + packed_offset(row, idx >> 1, nks) +
                                       (idx & 1) * 8);
  }
}

template <typename TX, int CH, bool PACK>
__global__ __launch_bounds__(256) void rowscale_kernel(const TX* __restrict__ X, _Float16* __restrict__ Y,
                                                       float* __restrict__ S, int M, int K, int texp) {
  constexpr int EPC = 16 / static_cast<int>(sizeof(TX));  // elements per 16-byte chunk
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int nks = packed_ksteps(K);
  if constexpr (PACK) {
    // Padding rows of the last 256-row block are zero; real rows zero their K tail below.
    if (row >= M) {
      if (row < (M + kPackRows - 1) / kPackRows * kPackRows)
        for (int oc = lane; oc < nks * 4; oc += kWave)
          *reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(Y) + packed_offset(row, oc, nks)) =
              u32x4{0u, 0u, 0u, 0u};
      return;
    }
    for (int oc = K / 8 + lane; oc < nks * 4; oc += kWave)
      *reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(Y) + packed_offset(row, oc, nks)) =
          u32x4{0u, 0u, 0u, 0u};
  }
  if (row >= M) return;  // wave-uniform; no barriers below
  const int nch = K / EPC;
  const u32x4* xr = reinterpret_cast<const u32x4*>(X + static_cast<size_t>(row) * K);

  u32x4 buf[CH];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = lane + c * kWave;
    buf[c] = idx < nch ? xr[idx] : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) amax = chunk_absmax(amax, buf[c], TX{});
  for (int idx = lane + CH * kWave; idx < nch; idx += kWave) amax = chunk_absmax(amax, xr[idx], TX{});
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));

  // Exponent from the bit fields; texp is log2(thresh).
  int e = 0;
  float sc = 1.f;
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

#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = lane + c * kWave;
    if (idx < nch) store_scaled(out_at<TX, PACK>(Y, row, K, idx, nks), buf[c], e, TX{});
  }
  for (int idx = lane + CH * kWave; idx < nch; idx += kWave)
    store_scaled(out_at<TX, PACK>(Y, row, K, idx, nks), xr[idx], e, TX{});
  if (lane == 0) S[row] = sc;
}

// thresh must be a positive, normal power of two; returns its exponent or a sentinel.
int thresh_exponent(float thresh) {
  uint32_t b;
  __builtin_memcpy(&b, &thresh, sizeof(b));
  const uint32_t ex = (b >> 23) & 0xffu;
  if ((b >> 31) != 0u || ex == 0u || ex == 0xffu || (b & 0x007fffffu) != 0u) return -1000;
  return static_cast<int>(ex) - 127;
}

template <typename TX, int CH, bool PACK>
int rowscale_launch(const void* X, void* Y, float* S, int M, int K, float thresh, void* stream) {
  if (M < 0 || K < 0 || K % 8 != 0) return G16_E_SHAPE;
  if (M == 0) return G16_OK;
  if (S == nullptr || (K > 0 && (X == nullptr || Y == nullptr))) return G16_E_NULL;
  if (!aligned16(X) || !aligned16(Y)) return G16_E_ALIGN;
  const int texp = thresh_exponent(thresh);
  if (texp == -1000) return G16_E_SHAPE;
  const int rows = PACK ? ceil_div(M, kPackRows) * kPackRows : M;
  const dim3 grid(ceil_div(rows, kRowsPerBlock)), block(256);
  return launch(rowscale_kernel<TX, CH, PACK>, grid, block, static_cast<hipStream_t>(stream),
                static_cast<const TX*>(X), static_cast<_Float16*>(Y), S, M, K, texp);
}

}  // namespace
}  // namespace g16

extern "C" int g16_rowscale_f32(const float* X, uint16_t* Y, float* S, int M, int K, float thresh, void* stream) {
  // 16 chunks of 4 floats per lane: rows up to K = 4096 are read once.
  return g16::rowscale_launch<float, 16, false>(X, Y, S, M, K, thresh, stream);
}

extern "C" int g16_rowscale_f16(const uint16_t* X, uint16_t* Y, float* S, int M, int K, float thresh, void* stream) {
  // 8 chunks of 8 halves per lane: rows up to K = 4096 are read once.
  return g16::rowscale_launch<_Float16, 8, false>(X, Y, S, M, K, thresh, stream);
}

extern "C" size_t g16_packed_a_bytes(int M, int K) {
  if (M <= 0 || K <= 0) return 0;
  return g16::packed_bytes_for(M, K);
}

extern "C" int g16_rowscale_pack_f32(const float* X, uint16_t* Yp, float* S, int M, int K, float thresh,
                                     void* stream) {
  return g16::rowscale_launch<float, 16, true>(X, Yp, S, M, K, thresh, stream);
}

extern "C" int g16_rowscale_pack_f16(const uint16_t* X, uint16_t* Yp, float* S, int M, int K, float thresh,
                                     void* stream) {
  return g16::rowscale_launch<_Float16, 8, true>(X, Yp, S, M, K, thresh, stream);
}
