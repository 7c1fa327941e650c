// Skinny GEMM on a strip-major copy of the weight (FastLinear's decode layout), 1 <= M <= 4.
//
// Semantics: those of the skinny path (reference: src/gtx16_fp16/kernels.py:153-219, ops.py:
// 45-51,78-84): fp32 math on the unquantised activations (fp32 or fp16 used as is), fp16 weights
// widened to fp32, bias added once, fp32 output.
//
// Layout. g16_pack_decode_weight writes w_t [K,N] as N/8 strips of 8 columns, each strip all K
// rows long and contiguous: D[s][k][0..7] = w_t[k][8s..8s+7] (16 bytes a row, K*16 bytes a strip;
// the same number of bytes as w_t, since N is a multiple of 8).
//
// Why. On the row-major weight a workgroup that streams whole 1 KB row segments owns 256 or 512
// columns, so with N = 4096 it must share K with 15 others and exchange partial sums through memory
// (skinny.hip): the arrival handshake and the last workgroup's read-back take ~2 us of a ~8.7 us
// M=1 4096x4096 call. Here a workgroup owns one strip over all of K, so no partial sum leaves the
// workgroup, and every load is still a coalesced 1 KB piece: lane l of a wavefront reads row k + l
// of the strip.
//
// Kernel: a workgroup (8 wavefronts) per strip. Wavefront w takes a contiguous run of rows (a
// multiple of 64); each lane multiplies its rows' 8 weights by its own activations (vector loads
// of A, which every workgroup reads from L2: M*K*4 bytes each, so the route pays for M <= 4 only),
// and issues its batch of U row loads before the first multiply. Reduction, fixed order: within a
// wavefront a butterfly that halves the columns each lane keeps at lane distances 32, 16 and 8,
// then full sums at distances 4, 2, 1 (each lane ends with one column); across the 8 wavefronts in
// wavefront order through LDS. Results are bitwise reproducible; they differ from skinny.hip's in
// the order of the fp32 additions only (both within the skinny path's tolerance of the fp64
// product).
#include "g16_common.hpp"

namespace g16 {
namespace {

constexpr int kStripWaves = 8;
constexpr int kStripThreads = kStripWaves * kWave;
constexpr int kStripCols = 8;

// One thread per 16-byte row piece of a strip: thread t of the grid writes D[s][k] for
// s = t / K, k = t % K, from the 16 bytes w_t[k][8s..8s+7]. The stores are coalesced, the loads
// 16-byte pieces of consecutive rows (a one-time copy per weight).
__global__ __launch_bounds__(256) void pack_decode_kernel(const _Float16* __restrict__ W, _Float16* __restrict__ D, int K,
                                                          int N, long total) {
  const long t = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const long s = t / K, k = t % K;
  *reinterpret_cast<u32x4*>(D + (s * K + k) * kStripCols) =
      *reinterpret_cast<const u32x4*>(W + k * N + s * kStripCols);
}

__device__ inline float act(const float* __restrict__ A, long i) { return A[i]; }
__device__ inline float act(const _Float16* __restrict__ A, long i) { return static_cast<float>(A[i]); }

template <typename TX, int MM, int U>
__global__ __launch_bounds__(kStripThreads) void strips_kernel(const TX* __restrict__ A, const _Float16* __restrict__ D,
                                                               float* __restrict__ C, const float* __restrict__ bias,
                                                               int N, int K, int rows_per_wave) {
  const int s = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k0 = wave * rows_per_wave;
  const int k1 = min(K, k0 + rows_per_wave);
  const _Float16* strip = D + static_cast<long>(s) * K * kStripCols;

  float acc[MM][8];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = 0.f;

  for (int r = k0; r < k1; r += kWave * U) {
    // Rows at or past k1 re-read the wavefront's last row (an in-bounds load) and contribute
    // nothing: both their weights and their activations are replaced by zeros, so the product is
    // 0 * 0 whatever the row holds (a +-inf or NaN weight or activation of the last row cannot leak
    // into the columns a second time).
    u32x4 w[U];
    float a[U][MM];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int row = min(r + kWave * u + lane, k1 - 1);
      w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(strip + static_cast<long>(row) * kStripCols));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = r + kWave * u + lane < k1;
      const int row = min(r + kWave * u + lane, k1 - 1);
#pragma unroll
      for (int m = 0; m < MM; ++m) a[u][m] = live ? act(A, static_cast<long>(m) * K + row) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = r + kWave * u + lane < k1;
      const uint32_t dw[4] = {live ? w[u].x : 0u, live ? w[u].y : 0u, live ? w[u].z : 0u, live ? w[u].w : 0u};
      float wf[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const half2v h = __builtin_bit_cast(half2v, dw[q]);
        wf[2 * q] = static_cast<float>(h.x);
        wf[2 * q + 1] = static_cast<float>(h.y);
      }
#pragma unroll
      for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(a[u][m], wf[j], acc[m][j]);
    }
  }

  // Wavefront reduction. At distance 32 the lower lanes keep columns 0-3 and the upper lanes 4-7,
  // each adding the partner's copy of the columns it keeps; then 2 of 4 at distance 16 and 1 of 2 at
  // distance 8. The 8 lanes that then hold the same column add up at distances 4, 2 and 1.
  const bool h5 = lane & 32, h4 = lane & 16, h3 = lane & 8;
  float v1[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    float v4[4], v2[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float send = h5 ? acc[m][j] : acc[m][j + 4];
      const float keep = h5 ? acc[m][j + 4] : acc[m][j];
      v4[j] = keep + __shfl_xor(send, 32);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float send = h4 ? v4[j] : v4[j + 2];
      const float keep = h4 ? v4[j + 2] : v4[j];
      v2[j] = keep + __shfl_xor(send, 16);
    }
    const float send = h3 ? v2[0] : v2[1];
    const float keep = h3 ? v2[1] : v2[0];
    v1[m] = keep + __shfl_xor(send, 8);
    v1[m] += __shfl_xor(v1[m], 4);
    v1[m] += __shfl_xor(v1[m], 2);
    v1[m] += __shfl_xor(v1[m], 1);
  }
  __shared__ float red[kStripWaves][MM][kStripCols];
  const int col = (h5 ? 4 : 0) + (h4 ? 2 : 0) + (h3 ? 1 : 0);
  if ((lane & 7) == 0) {
#pragma unroll
    for (int m = 0; m < MM; ++m) red[wave][m][col] = v1[m];
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < MM * kStripCols) {
    const int m = t / kStripCols, c = t % kStripCols;
    float sum = red[0][m][c];
#pragma unroll
    for (int w = 1; w < kStripWaves; ++w) sum += red[w][m][c];
    const int n = s * kStripCols + c;
    C[static_cast<long>(m) * N + n] = sum + (bias != nullptr ? bias[n] : 0.f);
  }
}

// Rows per wavefront: K spread over the 8 wavefronts in whole 64-row groups.
inline int strip_rows_per_wave(int K) { return ceil_div(ceil_div(K, kStripWaves), kWave) * kWave; }

template <typename TX, int U>
auto strips_fn_u(int M) {
  switch (M) {
    case 1: return strips_kernel<TX, 1, U>;
    case 2: return strips_kernel<TX, 2, U>;
    case 3: return strips_kernel<TX, 3, U>;
    default: return strips_kernel<TX, 4, U>;
  }
}

template <typename TX>
int strips_launch(const TX* A, const uint16_t* D, float* C, const float* bias, int M, int N, int K, void* stream) {
  if (M < 0 || N < 0 || K < 0 || M > G16_STRIPS_MAX_M || K % 8 != 0 || N % 8 != 0) return G16_E_SHAPE;
  if (M == 0 || N == 0) return G16_OK;
  if (C == nullptr || (K > 0 && (A == nullptr || D == nullptr))) return G16_E_NULL;
  if (!aligned16(A) || !aligned16(D) || !aligned16(C)) return G16_E_ALIGN;
  const int rows = strip_rows_per_wave(K);
  // Eight row loads per lane in flight when a wavefront has that many rows; K <= 2040 takes two.
  auto fn = rows >= 4 * kWave ? strips_fn_u<TX, 8>(M) : strips_fn_u<TX, 2>(M);
  return launch(fn, dim3(static_cast<unsigned>(N / kStripCols)), dim3(kStripThreads), static_cast<hipStream_t>(stream),
                A, reinterpret_cast<const _Float16*>(D), C, bias, N, K, rows);
}

}  // namespace
}  // namespace g16

extern "C" int g16_pack_decode_weight(const uint16_t* w_t, uint16_t* wd, int K, int N, void* stream) {
  if (K < 0 || N < 0 || K % 8 != 0 || N % 8 != 0) return G16_E_SHAPE;
  if (K == 0 || N == 0) return G16_OK;
  if (w_t == nullptr || wd == nullptr) return G16_E_NULL;
  if (!g16::aligned16(w_t) || !g16::aligned16(wd)) return G16_E_ALIGN;
  const long total = static_cast<long>(N / g16::kStripCols) * K;
  return g16::launch(g16::pack_decode_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256),
                     static_cast<hipStream_t>(stream), reinterpret_cast<const _Float16*>(w_t),
                     reinterpret_cast<_Float16*>(wd), K, N, total);
}

extern "C" int g16_skinny_strips_f32in(const float* A, const uint16_t* wd, float* C, const float* bias, int M, int N,
                                       int K, void* stream) {
  return g16::strips_launch<float>(A, wd, C, bias, M, N, K, stream);
}

extern "C" int g16_skinny_strips_f16in(const uint16_t* A, const uint16_t* wd, float* C, const float* bias, int M, int N,
                                       int K, void* stream) {
  return g16::strips_launch<_Float16>(reinterpret_cast<const _Float16*>(A), wd, C, bias, M, N, K, stream);
}

extern "C" int g16_skinny_strips_route(int M, int N, int K, int x_f32) {
  // Where the strip kernel beats the split kernel of skinny.hip on the same product (graph-timed,
  // weights streamed from HBM; M = 1..4, K and N from 768 to 14336): at M <= 2 on every shape
  // measured (4096 x 4096: 8.7 -> 7.3 us at M = 1; 1024 x 1024: 5.0 -> 3.0 us); at M = 3 and 4 up
  // to K * N = 2^22 (every workgroup reads all of A, M * K * 4 bytes, against K * 16 bytes of its
  // strip); past that with fp16 activations (half the bytes of A) at M = 3, and at M = 4 up to
  // N = 8192. fp32 activations at M = 3, 4 on larger weights stay on the split kernel (4096 x 4096,
  // M = 4: 10.1 against 11.1 us).
  if (M < 1 || M > G16_STRIPS_MAX_M || N <= 0 || K <= 0) return 0;
  if (M <= 2 || static_cast<long>(K) * N <= (1L << 22)) return 1;
  return !x_f32 && (M == 3 || N <= 8192);
}
