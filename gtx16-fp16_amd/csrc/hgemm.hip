// Tiled fp16 GEMM on the gfx950 matrix cores, fp32 accumulation, with an optional deterministic
// split over K.
//
// Semantics (reference: src/gtx16_fp16/kernels.py:35-151, ops.py:92-108):
//   C[M,N] = rscale[row] * (A[M,K] @ B[K,N]) + bias[N], cast to fp32 or fp16 (nearest-even),
// scale first, then bias, then cast (kernels.py:116-133). A is the fp16 output of the rowscale
// cast (K contiguous), B the fp16 weight w_t (N contiguous).
//
// Structure:
//   * 256 threads = 4 wavefronts per workgroup; a workgroup owns a BM x BN output tile, each
//     wavefront a (BM/WGM) x (BN/WGN) sub-tile made of 32x32 blocks computed with
//     v_mfma_f32_32x32x16_f16 (fp32 accumulators).
//   * K advances in steps of BK = 64 through a two-stage LDS ring: the global loads for step k+1
//     are issued before the MFMAs of step k and land in the other stage after them, one barrier
//     per step.
//   * MFMA operands need K-contiguous runs per lane for both A and B. A tiles are copied as is
//     ([row][k]); B tiles ([k][n] in memory) are transposed in registers while staging (each
//     thread loads KR rows x 8 columns and writes 8 runs of KR halves), so LDS holds [n][k].
//   * LDS rows are 64 halves (128 bytes, 8 chunks of 16 bytes); chunk c of row r is stored at
//     chunk c ^ swizzle(r), which keeps the 16-byte fragment reads and the staging writes free of
//     bank conflicts.
//   * Tiles are assigned XCD-aware: the hardware deals workgroups round-robin over the 8 XCDs, so
//     workgroup b is mapped to tile (b % 8) * (T / 8) + b / 8, giving each XCD a contiguous run
//     of tiles, which a grouped (GROUP_M rows at a time) order turns into a compact 2-D block
//     that shares A rows and B columns in that XCD's L2.
//   * Split-K: slice z of tile t covers K range [z*kchunk, (z+1)*kchunk). Every slice stores its
//     fp32 accumulators to the workspace in the lanes' own register order (fully coalesced 16-byte
//     stores); the last slice to arrive adds all slices in slice order and runs the epilogue.
//     Deterministic, and bias/scale/cast are fused (the reference prefills C with the bias and
//     adds with fp32 atomics, kernels.py:119-122, ops.py:54-62).
#include "g16_common.hpp"

namespace g16 {
namespace {

constexpr int BK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;

template <int BM_, int BN_, int WGM_, int WGN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
  static_assert(WGM * WGN == 4, "4 wavefronts per workgroup");
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wavefront sub-tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;      // 32x32 MFMA blocks per wavefront
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "32x32 blocks");
  static constexpr int A_CH = BM * BK / 8 / kThreads;  // 16-byte A chunks per thread
  static constexpr int KR = BK * BN / (kThreads * 8);   // B rows per thread (8 columns each)
  static_assert(A_CH >= 1 && (KR == 2 || KR == 4 || KR == 8), "staging shape");
  static constexpr int NB = BN / 8;  // 8-column groups per B row
  static constexpr int LDS_HALVES = 2 * (BM + BN) * BK;
};

using Cfg256 = TileCfg<256, 256, 2, 2>;
using Cfg128 = TileCfg<128, 128, 2, 2>;
using Cfg64 = TileCfg<64, 128, 1, 4>;
using Cfg32 = TileCfg<32, 128, 1, 4>;

__device__ inline int swz_a(int row) { return row & 7; }
__device__ inline int swz_b(int n) { return (n & 7) ^ ((n >> 3) & 7); }

// Halves (hi16 of one dword, lo16 of another) packers for the B transpose.
__device__ inline uint32_t pick(uint32_t lo_src, uint32_t hi_src, bool odd) {
  return odd ? ((lo_src >> 16) | (hi_src & 0xffff0000u)) : ((lo_src & 0xffffu) | (hi_src << 16));
}

template <class Cfg, bool OUT_F16, bool SPLITK>
__global__ __launch_bounds__(kThreads) void hgemm_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                                                         void* __restrict__ Cv, const float* __restrict__ bias,
                                                         const float* __restrict__ rscale, float* __restrict__ part,
                                                         uint32_t* __restrict__ counters, int M, int N, int K,
                                                         int kchunk, int ksplit, int ntm, int ntn) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, TM = Cfg::TM, TN = Cfg::TN, KR = Cfg::KR, NB = Cfg::NB;
  __shared__ __attribute__((aligned(16))) _Float16 smem[Cfg::LDS_HALVES];
  _Float16* const As = smem;                 // [2][BM][BK]
  _Float16* const Bs = smem + 2 * BM * BK;   // [2][BN][BK]

  // ---- tile assignment (XCD-aware, grouped) ----
  const int ntiles = ntm * ntn;
  int lin = blockIdx.x;
  if (ntiles % 8 == 0) lin = (lin % 8) * (ntiles / 8) + lin / 8;
  const int per_group = kGroupM * ntn;
  const int first_m = (lin / per_group) * kGroupM;
  const int gsz = min(ntm - first_m, kGroupM);
  const int tm = first_m + (lin % per_group) % gsz;
  const int tn = (lin % per_group) / gsz;
  const int tile = tm * ntn + tn;
  const int m0 = tm * BM, n0 = tn * BN;
  const int z = blockIdx.y;
  const int kbeg = z * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const int nk = kend > kbeg ? ceil_div(kend - kbeg, BK) : 0;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / Cfg::WGN) * Cfg::WTM;
  const int wn0 = (wave % Cfg::WGN) * Cfg::WTN;

  // ---- global -> register staging ----
  u32x4 ra[Cfg::A_CH];
  u32x4 rb[KR];
  const int a_c = tid & 7;    // 16-byte chunk within the 64-half row
  const int a_r = tid >> 3;   // rows a_r + 32*i
  const int b_nb = tid % NB;  // 8-column group
  const int b_kb = tid / NB;  // rows b_kb*KR .. +KR-1

  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < Cfg::A_CH; ++i) {
      const int row = m0 + a_r + 32 * i;
      const int kk = k0 + a_c * 8;
      ra[i] = (row < M && kk < kend) ? *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(row) * K + kk)
                                     : u32x4{0u, 0u, 0u, 0u};
    }
    const int col = n0 + b_nb * 8;
#pragma unroll
    for (int j = 0; j < KR; ++j) {
      const int kr = k0 + b_kb * KR + j;
      rb[j] = (kr < kend && col < N) ? *reinterpret_cast<const u32x4*>(B + static_cast<size_t>(kr) * N + col)
                                     : u32x4{0u, 0u, 0u, 0u};
    }
  };

  auto swrite = [&](int stage) {
    _Float16* as = As + stage * BM * BK;
    _Float16* bs = Bs + stage * BN * BK;
#pragma unroll
    for (int i = 0; i < Cfg::A_CH; ++i) {
      const int row = a_r + 32 * i;
      *reinterpret_cast<u32x4*>(as + row * BK + ((a_c ^ swz_a(row)) * 8)) = ra[i];
    }
    const int kl = b_kb * KR;
    const int chunk = kl / 8, sub = kl % 8;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int nl = b_nb * 8 + n;
      _Float16* dst = bs + nl * BK + ((chunk ^ swz_b(nl)) * 8) + sub;
      const int dw = n >> 1;
      const bool odd = (n & 1) != 0;
      uint32_t w[KR / 2];
#pragma unroll
      for (int p = 0; p < KR / 2; ++p) w[p] = pick(rb[2 * p][dw], rb[2 * p + 1][dw], odd);
      if constexpr (KR == 8) {
        *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
      } else if constexpr (KR == 4) {
        *reinterpret_cast<u32x2*>(dst) = u32x2{w[0], w[1]};
      } else {
        *reinterpret_cast<uint32_t*>(dst) = w[0];
      }
    }
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

  const int frow = lane & 31;  // fragment row (A) / column (B) within a 32-block
  const int fk = lane >> 5;    // which 8-run of the 16-wide K step

  if (nk > 0) {
    gload(kbeg);
    swrite(0);
  }
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const int cur = it & 1;
    if (it + 1 < nk) gload(kbeg + (it + 1) * BK);
    const _Float16* as = As + cur * BM * BK;
    const _Float16* bs = Bs + cur * BN * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = ks * 2 + fk;
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm0 + 32 * i + frow;
        af[i] = *reinterpret_cast<const half8*>(as + row * BK + ((chunk ^ swz_a(row)) * 8));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = wn0 + 32 * j + frow;
        bf[j] = *reinterpret_cast<const half8*>(bs + n * BK + ((chunk ^ swz_b(n)) * 8));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (it + 1 < nk) swrite(cur ^ 1);
    __syncthreads();
  }

  // ---- split-K: publish this slice, let the last slice reduce ----
  if constexpr (SPLITK) {
    constexpr uint32_t TILE_BYTES = BM * BN * 4;
    const __amdgpu_buffer_rsrc_t slices =
        coherent_rsrc(part + static_cast<size_t>(tile) * ksplit * (BM * BN), static_cast<uint32_t>(ksplit) * TILE_BYTES);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t slot = (((wave * TM + i) * TN + j) * 4 + q) * 64 + lane;
          store_coherent4(slices, static_cast<uint32_t>(z) * TILE_BYTES + slot * 16u,
                          float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
        }
    if (!arrive_last_coherent(counters + tile * kCounterStride, static_cast<uint32_t>(ksplit))) return;
    // Slices are added in slice order, ZB slices' loads in flight at a time (every slice, this
    // one's included, is read back from the workspace).
    constexpr int SLOTS = TM * TN * 4;
    constexpr int ZB = (128 / (SLOTS * 4)) < 1 ? 1 : ((128 / (SLOTS * 4)) > 8 ? 8 : (128 / (SLOTS * 4)));
    float4v sum[SLOTS];
#pragma unroll
    for (int q = 0; q < SLOTS; ++q) sum[q] = float4v{0.f, 0.f, 0.f, 0.f};
    for (int z0 = 0; z0 < ksplit; z0 += ZB) {
      float4v v[ZB][SLOTS];
#pragma unroll
      for (int b = 0; b < ZB; ++b)
#pragma unroll
        for (int q = 0; q < SLOTS; ++q) {
          const uint32_t slot = static_cast<uint32_t>((wave * SLOTS + q) * 64 + lane);
          v[b][q] = z0 + b < ksplit ? load_coherent4(slices, static_cast<uint32_t>(z0 + b) * TILE_BYTES + slot * 16u)
                                    : float4v{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int b = 0; b < ZB; ++b)
#pragma unroll
        for (int q = 0; q < SLOTS; ++q)
          if (z0 + b < ksplit) sum[q] += v[b][q];
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4v t = sum[(i * TN + j) * 4 + q];
          acc[i][j][4 * q] = t.x;
          acc[i][j][4 * q + 1] = t.y;
          acc[i][j][4 * q + 2] = t.z;
          acc[i][j][4 * q + 3] = t.w;
        }
    reset_counter(counters + tile * kCounterStride);
  }

  // ---- epilogue: C = rscale[row] * acc + bias[col] ----
  // 32x32 accumulator layout: lane l, register r -> column l % 32, row 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm0 + 32 * i + 8 * (r >> 2) + 4 * fk + (r & 3);
      if (row >= M) continue;
      const float rs = rscale != nullptr ? rscale[row] : 1.f;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn0 + 32 * j + frow;
        if (col >= N) continue;
        const float v = acc[i][j][r] * rs + (bias != nullptr ? bias[col] : 0.f);
        if constexpr (OUT_F16) {
          static_cast<_Float16*>(Cv)[static_cast<size_t>(row) * N + col] = static_cast<_Float16>(v);
        } else {
          static_cast<float*>(Cv)[static_cast<size_t>(row) * N + col] = v;
        }
      }
    }
  }
}

enum class Tile { T256, T128, T64, T32 };

struct Plan {
  Tile tile;
  int bm, bn;
  int ntm, ntn;
};

// Split-K launches use the tiles up to 128x128 (the 256x256 tile has no split-K variant: its
// accumulators fill the register file).
Plan choose_tile(int M, int N, bool splitk) {
  Plan p{};
  if (M <= 32) {
    p.tile = Tile::T32; p.bm = 32; p.bn = 128;
  } else if (M <= 64) {
    p.tile = Tile::T64; p.bm = 64; p.bn = 128;
  } else if (!splitk && M >= 1024 && N >= 256 && static_cast<long>(ceil_div(M, 256)) * ceil_div(N, 256) >= 128) {
    p.tile = Tile::T256; p.bm = 256; p.bn = 256;
  } else {
    p.tile = Tile::T128; p.bm = 128; p.bn = 128;
  }
  p.ntm = ceil_div(M, p.bm);
  p.ntn = ceil_div(N, p.bn);
  return p;
}

struct KSplit {
  int ksplit;
  int kchunk;
};

KSplit ksplit_for(int K, int ksplit) {
  if (K <= 0 || ksplit <= 1) return {1, K > 0 ? K : 0};
  const int kchunk = ceil_div(ceil_div(K, ksplit), BK) * BK;
  return {ceil_div(K, kchunk), kchunk};
}

template <bool OUT_F16>
using GemmFn = void (*)(const _Float16*, const _Float16*, void*, const float*, const float*, float*, uint32_t*, int,
                        int, int, int, int, int, int);

template <bool OUT_F16>
GemmFn<OUT_F16> gemm_fn(Tile t, bool splitk) {
  if (splitk) {
    switch (t) {
      case Tile::T128: return hgemm_kernel<Cfg128, OUT_F16, true>;
      case Tile::T64: return hgemm_kernel<Cfg64, OUT_F16, true>;
      default: return hgemm_kernel<Cfg32, OUT_F16, true>;
    }
  }
  switch (t) {
    case Tile::T256: return hgemm_kernel<Cfg256, OUT_F16, false>;
    case Tile::T128: return hgemm_kernel<Cfg128, OUT_F16, false>;
    case Tile::T64: return hgemm_kernel<Cfg64, OUT_F16, false>;
    default: return hgemm_kernel<Cfg32, OUT_F16, false>;
  }
}

size_t splitk_ws_bytes(const Plan& p, int ksplit) {
  if (ksplit <= 1) return 0;
  const size_t ntiles = static_cast<size_t>(p.ntm) * p.ntn;
  return ntiles * ksplit * static_cast<size_t>(p.bm) * p.bn * sizeof(float);
}

size_t splitk_counter_bytes(const Plan& p, int ksplit) {
  if (ksplit <= 1) return 0;
  return counter_bytes(static_cast<size_t>(p.ntm) * p.ntn);
}

int gemm_launch(const uint16_t* A, const uint16_t* B, void* C, bool out_f16, const float* bias, const float* rscale,
                int M, int N, int K, int ksplit, void* ws, size_t ws_bytes, uint32_t* counters_in,
                size_t counter_bytes_in, void* stream) {
  if (M < 0 || N < 0 || K < 0 || K % 8 != 0 || N % 8 != 0) return G16_E_SHAPE;
  if (M == 0 || N == 0) return G16_OK;
  if (ksplit < 1 || ksplit > 256) return G16_E_SPLIT;
  if (C == nullptr || (K > 0 && (A == nullptr || B == nullptr))) return G16_E_NULL;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return G16_E_ALIGN;
  const KSplit ks = ksplit_for(K, ksplit);
  const Plan p = choose_tile(M, N, ks.ksplit > 1);
  float* part = nullptr;
  uint32_t* counters = nullptr;
  if (ks.ksplit > 1) {
    if (ws == nullptr || ws_bytes < splitk_ws_bytes(p, ks.ksplit)) return G16_E_WORKSPACE;
    if (counters_in == nullptr || counter_bytes_in < splitk_counter_bytes(p, ks.ksplit)) return G16_E_WORKSPACE;
    if (!aligned16(ws) || !aligned16(counters_in)) return G16_E_ALIGN;
    counters = counters_in;
    part = static_cast<float*>(ws);
  }
  const dim3 grid(static_cast<unsigned>(p.ntm * p.ntn), static_cast<unsigned>(ks.ksplit)), block(kThreads);
  const auto* a = reinterpret_cast<const _Float16*>(A);
  const auto* b = reinterpret_cast<const _Float16*>(B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool sk = ks.ksplit > 1;
  if (out_f16)
    return launch(gemm_fn<true>(p.tile, sk), grid, block, s, a, b, C, bias, rscale, part, counters, M, N, K, ks.kchunk,
                  ks.ksplit, p.ntm, p.ntn);
  return launch(gemm_fn<false>(p.tile, sk), grid, block, s, a, b, C, bias, rscale, part, counters, M, N, K, ks.kchunk,
                ks.ksplit, p.ntm, p.ntn);
}

}  // namespace
}  // namespace g16

extern "C" int g16_hgemm_plan(int M, int N, int K, int num_cus) {
  // Split K when the output tiles cannot give every CU a workgroup, keeping >= 256 K per slice.
  if (M <= 0 || N <= 0 || K <= 0 || num_cus <= 0) return 1;
  const g16::Plan p = g16::choose_tile(M, N, false);
  const int tiles = p.ntm * p.ntn;
  if (tiles >= num_cus / 2 || K < 512) return 1;
  const g16::Plan q = g16::choose_tile(M, N, true);
  const int qtiles = q.ntm * q.ntn;
  if (qtiles != tiles) return 1;
  int ks = g16::ceil_div(num_cus, tiles);
  const int cap = K / 256;
  ks = ks > cap ? cap : ks;
  ks = ks > 256 ? 256 : ks;
  return g16::ksplit_for(K, ks < 1 ? 1 : ks).ksplit;
}

extern "C" size_t g16_hgemm_splitk_workspace_bytes(int M, int N, int K, int ksplit) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const g16::KSplit ks = g16::ksplit_for(K, ksplit);
  const g16::Plan p = g16::choose_tile(M, N, ks.ksplit > 1);
  return g16::splitk_ws_bytes(p, ks.ksplit);
}

extern "C" size_t g16_hgemm_splitk_counter_bytes(int M, int N, int K, int ksplit) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const g16::KSplit ks = g16::ksplit_for(K, ksplit);
  const g16::Plan p = g16::choose_tile(M, N, ks.ksplit > 1);
  return g16::splitk_counter_bytes(p, ks.ksplit);
}

extern "C" int g16_hgemm_f32out(const uint16_t* A, const uint16_t* B, float* C, const float* bias, const float* rscale,
                                int M, int N, int K, void* stream) {
  return g16::gemm_launch(A, B, C, false, bias, rscale, M, N, K, 1, nullptr, 0, nullptr, 0, stream);
}

extern "C" int g16_hgemm_f16out(const uint16_t* A, const uint16_t* B, uint16_t* C, const float* bias,
                                const float* rscale, int M, int N, int K, void* stream) {
  return g16::gemm_launch(A, B, C, true, bias, rscale, M, N, K, 1, nullptr, 0, nullptr, 0, stream);
}

extern "C" int g16_hgemm_splitk(const uint16_t* A, const uint16_t* B, void* C, int c_is_f16, const float* bias,
                                const float* rscale, int M, int N, int K, int ksplit, void* workspace,
                                size_t workspace_bytes, uint32_t* counters, size_t counter_bytes, void* stream) {
  return g16::gemm_launch(A, B, C, c_is_f16 != 0, bias, rscale, M, N, K, ksplit, workspace, workspace_bytes, counters,
                          counter_bytes, stream);
}
