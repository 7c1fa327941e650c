// Weight packing for the 256x256 GEMM (FastLinear's prepacked weight).
//
// The weight w_t is [K,N] with N contiguous, as the reference stores it (src/gtx16_fp16/linear.py:
// 27-37). Its MFMA B operand needs runs along K, so with the row-major weight the GEMM reads B
// fragments through the LDS transposing read, which costs about twice a plain 16-byte read per
// byte. g16_pack_weight writes w_t^T ([N,K]) once in the tile-packed layout of g16_common.hpp:
// the GEMM then copies contiguous 16 KB stage images of B and reads its fragments like A's.
//
// One thread per 16-byte output chunk: 64 threads take 64 consecutive columns n of one 8-row group
// of w_t, so each of the 8 loads is a coalesced 128-byte row piece; the chunk is stored at its packed
// offset. Columns past N (up to the 256-column block) and rows past K are written as zeros.
#include "g16_common.hpp"

namespace g16 {
namespace {

__global__ __launch_bounds__(256) void pack_weight_kernel(const _Float16* __restrict__ W, unsigned char* __restrict__ P,
                                                          int K, int N, int nks) {
  const int n = blockIdx.x * 64 + (threadIdx.x & 63);  // row of w^T, < ceil(N/256)*256 by the grid
  const int oc = blockIdx.y * 4 + (threadIdx.x >> 6);  // 8-column group of K
  if (oc >= nks * 4) return;
  half8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = oc * 8 + e;
    v[e] = (n < N && k < K) ? W[static_cast<size_t>(k) * N + n] : static_cast<_Float16>(0.f);
  }
  *reinterpret_cast<half8*>(P + packed_offset(n, oc, nks)) = v;
}

}  // namespace
}  // namespace g16

extern "C" size_t g16_packed_b_bytes(int K, int N) {
  if (K <= 0 || N <= 0) return 0;
  return g16::packed_bytes_for(N, K);
}

extern "C" int g16_pack_weight(const uint16_t* w_t, uint16_t* wp, int K, int N, void* stream) {
  if (K < 0 || N < 0 || K % 8 != 0 || N % 8 != 0) return G16_E_SHAPE;
  if (K == 0 || N == 0) return G16_OK;
  if (w_t == nullptr || wp == nullptr) return G16_E_NULL;
  if (!g16::aligned16(w_t) || !g16::aligned16(wp)) return G16_E_ALIGN;
  const int nks = g16::packed_ksteps(K);
  const int rows = g16::ceil_div(N, g16::kPackRows) * g16::kPackRows;
  const dim3 grid(static_cast<unsigned>(rows / 64), static_cast<unsigned>(nks)), block(256);
  return g16::launch(g16::pack_weight_kernel, grid, block, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const _Float16*>(w_t), reinterpret_cast<unsigned char*>(wp), K, N, nks);
}
