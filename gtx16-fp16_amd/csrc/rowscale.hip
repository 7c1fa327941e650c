// Row rescale + fp16 cast for the quantised GEMM path (M > 8).
//
// Semantics (reference: src/gtx16_fp16/kernels.py:227-250, called from ops.py:86-90): see
// rowscale_math.hpp, which holds the arithmetic (shared with the GEMM kernels that cast their own
// activations).
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
#include "rowscale_math.hpp"

namespace g16 {
namespace {

constexpr int kRowsPerBlock = 4;

__device__ inline void store_scaled(_Float16* y, u32x4 v, int e, float) {
  *reinterpret_cast<u32x2*>(y) = cast_scaled(v, e, float{});
}
__device__ inline void store_scaled(_Float16* y, u32x4 v, int e, _Float16) {
  *reinterpret_cast<u32x4*>(y) = cast_scaled(v, e, _Float16{});
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

  int e;
  float sc;
  row_exponent(amax, texp, e, sc);

#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = lane + c * kWave;
    if (idx < nch) store_scaled(out_at<TX, PACK>(Y, row, K, idx, nks), buf[c], e, TX{});
  }
  for (int idx = lane + CH * kWave; idx < nch; idx += kWave)
    store_scaled(out_at<TX, PACK>(Y, row, K, idx, nks), xr[idx], e, TX{});
  if (lane == 0) S[row] = sc;
}

// Whole rows of exactly 64 * CH chunks (K = 4096 for both input types), and no padding rows:
// every wavefront casts two rows, r and r + M / 2, and issues the second row's loads before the
// first row's stores, with no per-chunk conditions. Same arithmetic and stores as above
// (4096 x 4096 fp32 into the packed layout, event-timed on one box: 16.35 -> 15.75 us alone,
// 120.85 -> 120.41 us per (cast, GEMM) pair of mm_t, medians of 8 alternating batches).
template <typename TX, int CH, bool PACK>
__global__ __launch_bounds__(256) void rowscale_rows2_kernel(const TX* X, _Float16* Y, float* S, int M, int K, int texp) {
  const int lane = threadIdx.x & (kWave - 1);
  const int nks = packed_ksteps(K);
  const int half = M / 2;
  const int r0 = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  auto load = [&](int row, u32x4 (&buf)[CH]) {
    const u32x4* xr = reinterpret_cast<const u32x4*>(X + static_cast<size_t>(row) * K);
#pragma unroll
    for (int c = 0; c < CH; ++c) buf[c] = xr[lane + c * kWave];
  };
  auto finish = [&](int row, const u32x4 (&buf)[CH]) {
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) amax = chunk_absmax(amax, buf[c], TX{});
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    int e;
    float sc;
    row_exponent(amax, texp, e, sc);
#pragma unroll
    for (int c = 0; c < CH; ++c) store_scaled(out_at<TX, PACK>(Y, row, K, lane + c * kWave, nks), buf[c], e, TX{});
    if (lane == 0) S[row] = sc;
  };
  u32x4 a[CH], b[CH];
  load(r0, a);
  load(r0 + half, b);
  finish(r0, a);
  finish(r0 + half, b);
}

template <typename TX, int CH, bool PACK>
int rowscale_launch(const void* X, void* Y, float* S, int M, int K, float thresh, void* stream) {
  if (M < 0 || K < 0 || K % 8 != 0) return G16_E_SHAPE;
  if (M == 0) return G16_OK;
  if (S == nullptr || (K > 0 && (X == nullptr || Y == nullptr))) return G16_E_NULL;
  if (!aligned16(X) || !aligned16(Y)) return G16_E_ALIGN;
  const int texp = thresh_exponent(thresh);
  if (texp == -1000) return G16_E_SHAPE;
  constexpr int EPC = 16 / static_cast<int>(sizeof(TX));
  if (K == kWave * CH * EPC && M % (2 * kRowsPerBlock) == 0 && (!PACK || M % kPackRows == 0)) {
    // whole rows, an even number of workgroup row sets, no padding rows: the two-row form
    return launch(rowscale_rows2_kernel<TX, CH, PACK>, dim3(M / (2 * kRowsPerBlock)), dim3(256),
                  static_cast<hipStream_t>(stream), static_cast<const TX*>(X), static_cast<_Float16*>(Y), S, M, K,
                  texp);
  }
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
