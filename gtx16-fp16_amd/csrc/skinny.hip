// Skinny GEMM for 1 <= M <= 8 (token-by-token decode): C[M,N] = A[M,K] @ B[K,N] + bias.
//
// Semantics (reference: src/gtx16_fp16/kernels.py:153-219, ops.py:45-51,78-84): fp32 math on the
// unquantised activations (fp32 or fp16 used as is), fp16 weights widened to fp32, bias added once,
// fp32 output.
//
// The path is HBM-bound for small M (arithmetic intensity <= 8 flop/byte): B is streamed exactly
// once and the design follows from B's layout ([K,N], N contiguous):
//   * A workgroup (8 wavefronts) owns a strip of B's columns and a slice of K rows. Each wavefront
//     takes a contiguous run of rows, and one load instruction reads 1 KB of them: one 1 KB row
//     segment with 512-column strips, two 512-byte row segments (lanes 0-31 row k, lanes 32-63
//     row k+1) with 256-column strips; 16 bytes = 8 fp16 columns a lane. Every load is fully
//     coalesced and the activations A[m,k] (and A[m,k+1]) it multiplies are the same for the
//     whole wavefront: A comes in through scalar loads, and the vector memory path carries
//     nothing but B.
//   * Each lane issues its batch of row loads before it uses any, so a workgroup has tens of KB
//     of B in flight: enough to cover HBM latency with up to one workgroup per CU. The weight is
//     read exactly once, so the loads are non-temporal (measured 7-8 % faster at 4096x4096).
//   * Reduction is fixed-order: the partial rows are added in order through LDS; when K is split
//     over several workgroups, each slice publishes its strip x M partial with device-coherent
//     stores and the last slice to arrive (per strip) adds the slices in slice order. No
//     floating-point atomics: results are bitwise reproducible and C needs no zero-fill (the
//     reference zero-fills C and accumulates with atomicAdd, kernels.py:205-206).
//   * Strip width: for a given grid (about one workgroup per CU) it sets how many slices share a
//     strip, and the last arriver reads slices x M x width partial sums back through one CU.
//     Up to N = 8192 the strips are 256 columns (half the slices of 512-column strips and a 4x
//     smaller read-back; 128-column strips stream worse: 1 x 4096^2 in 8.58-8.62 us, against
//     9.11-9.16 with 512 columns and 8.91-8.98 with 128), above that 512 (strip_cols).
#include <mutex>
#include <type_traits>

#include "g16_common.hpp"

namespace g16 {

// Split buffers of g16_skinny_f32in_noalloc: the arrival counters in the first
// G16_NOALLOC_COUNTER_BYTES, the fp32 partials in the next G16_NOALLOC_PARTIAL_BYTES. A file-scope
// device array, so every GPU the library runs on holds its own copy until the process ends; host
// code reaches it only through the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[G16_NOALLOC_COUNTER_BYTES + G16_NOALLOC_PARTIAL_BYTES];

namespace {

constexpr int kWaves = 8;        // wavefronts per workgroup
constexpr int kThreads = kWaves * kWave;
constexpr int kMinRows = 8;      // the plan gives every wavefront at least this many rows
constexpr int kMfBatch = 32;     // K rows per batch of the matrix-core form
constexpr int kMfMaxBatches = 4; // ... its activations held in registers: up to 128 rows per wavefront

// Launch schedule of the kernel:
//   cols   -- columns of the strip a workgroup owns: 512 (one 1 KB row per load instruction) or
//             256 (two 512-byte rows per load instruction, lanes 0-31 and 32-63);
//   loads  -- load instructions each lane issues per batch (loads x 1 KB per wavefront in flight);
//   issue  -- a scheduling barrier after the batch's loads, so all of them are issued before the
//             first multiply (the compiler otherwise starts waiting on the first load part-way
//             through the batch);
//   uncond -- the split reduction's partial loads are issued unconditionally (a lane with nothing
//             to add reads a valid slot and drops it) instead of under a per-lane condition.
template <int COLS, int LOADS, bool ISSUE, bool UNCOND>
struct Sched {
  static constexpr int cols = COLS, loads = LOADS;
  static constexpr bool issue = ISSUE, uncond = UNCOND;
  static constexpr int lanes_per_row = COLS / 8;
  static constexpr int rows_per_load = kWave / lanes_per_row;
  static constexpr int parts = kWaves * rows_per_load;  // partial rows a workgroup reduces in LDS
  static_assert(COLS == 256 || COLS == 512, "strip width");
};

// The plan's unit of whole blocks per wavefront: 16 rows.
constexpr int kPlanBlockRows = 16;

__device__ inline float x_at(const float* __restrict__ A, size_t i) { return A[i]; }
// fp16 activations are read as the aligned dword holding them, so the (wavefront-uniform) load
// stays a scalar load.
__device__ inline float x_at(const _Float16* __restrict__ A, size_t i) {
  const uint32_t d = reinterpret_cast<const uint32_t*>(A)[i >> 1];
  const half2v h = __builtin_bit_cast(half2v, d);
  return static_cast<float>((i & 1) ? h.y : h.x);
}

template <int MM>
__device__ inline void fma_row(float (&acc)[MM][8], const float (&a)[MM], u32x4 w) {
  float wf[8];
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const half2v h = __builtin_bit_cast(half2v, d[q]);
    wf[2 * q] = static_cast<float>(h.x);
    wf[2 * q + 1] = static_cast<float>(h.y);
  }
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(a[m], wf[j], acc[m][j]);
}

// Two fp16 parts of a finite x (|x| < 2^15 after the row scaling): hi is x rounded toward zero to
// fp16, lo the rest rounded to nearest, so |x - hi - lo| <= 2^-21 |x| (<= 2^-25 where lo is
// subnormal), and an fp16 x gives hi = x. Both parts carry x's sign: a part that would be zero for
// a nonzero x is the smallest subnormal (2^-24) with x's sign instead (an error of <= 2^-23,
// negligible next to a row whose largest |x| is >= 2^14). An infinite weight times (hi, lo)
// therefore gives the infinity the fp32 product gives, never inf - inf; x = +-0 gives (+-0, 0), and
// 0 * inf is NaN either way.
__device__ inline void split_hi_lo(float x, _Float16& hi, _Float16& lo) {
  const uint16_t tiny = static_cast<uint16_t>(((__float_as_uint(x) >> 16) & 0x8000u) | 1u);
  uint16_t hb = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  hb -= fabsf(static_cast<float>(__builtin_bit_cast(_Float16, hb))) > fabsf(x) ? 1 : 0;  // toward zero
  const uint16_t lb = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x - static_cast<float>(__builtin_bit_cast(_Float16, hb))));
  const bool hz = (hb & 0x7fffu) == 0, xz = x == 0.f;
  hi = __builtin_bit_cast(_Float16, hz ? (xz ? hb : tiny) : hb);
  lo = __builtin_bit_cast(_Float16, hz ? (xz ? static_cast<uint16_t>(0u) : tiny) : ((lb & 0x7fffu) == 0 ? tiny : lb));
}

// MF (launched by use_mf: M = 8, 256-column strips, 32..128 K rows per wavefront): a wavefront
// whose activations are all finite multiplies on the matrix cores (below); one with an inf or NaN
// among them takes the fp32 FMA loop.
template <typename TX, int MM, class S, bool MF = false>
__global__ __launch_bounds__(kThreads) void skinny_kernel(const TX* __restrict__ A, const _Float16* __restrict__ B,
                                                          float* __restrict__ C, const float* __restrict__ bias,
                                                          float* __restrict__ part, uint32_t* __restrict__ counters,
                                                          int N, int K, int rows_per_wave, int ksplit, int nstrips) {
  constexpr int kStripCols = S::cols, kLanesPerRow = S::lanes_per_row, kRowsPerLoad = S::rows_per_load;
  // Partial sums of every (wavefront, row of its load instructions) pair: 16 KB per row of A.
  constexpr int kParts = S::parts;
  __shared__ float red[kParts][MM][kStripCols];
  const int strip = blockIdx.x % nstrips;
  const int kpart = blockIdx.x / nstrips;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane / kLanesPerRow;  // which row of a load instruction this lane reads
  const int lcol = (lane % kLanesPerRow) * 8;
  const int col = strip * kStripCols + lcol;
  const int k0 = (kpart * kWaves + wave) * rows_per_wave;
  const int k1 = min(K, k0 + rows_per_wave);

  float acc[MM][8];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = 0.f;

  // A[m, r] for row r = k + sub of a load instruction that starts at row k: the instruction's
  // kRowsPerLoad activations are wavefront-uniform (scalar loads), each lane keeps its own. Rows at
  // or past k1 are not read (tail of the slice) and give 0.
  auto act = [&](int k, bool whole, float (&a)[MM]) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      float v[kRowsPerLoad];
#pragma unroll
      for (int r = 0; r < kRowsPerLoad; ++r)
        v[r] = (whole || k + r < k1) ? x_at(A, static_cast<size_t>(m) * K + k + r) : 0.f;
      a[m] = v[0];
#pragma unroll
      for (int r = 1; r < kRowsPerLoad; ++r) a[m] = sub == r ? v[r] : a[m];
    }
  };

  // Matrix-core form (MF): one v_mfma_f32_16x16x32_f16 computes 16 A rows x 16 columns x 32 K
  // rows. Its A rows 0-7 are the fp16 hi parts of the (row-scaled) activations, rows 8-15 their lo
  // parts (split_hi_lo), so C[m] + C[m + 8] is the fp32-accurate product for m < 8: the products
  // of fp16 parts are exact, and the fp32 FMAs per weight and row become ~100 VALU instructions per
  // 32 rows. Each row m is scaled by 2^-e_m (exact) so its largest |x| over the wavefront's rows
  // lies in [2^14, 2^15), and the partial sum is scaled back by 2^e_m.
  //   A batch is 32 K rows (16 loads: lanes 0-31 row r + 2u, lanes 32-63 row r + 2u + 1, 8 columns
  // each, as in the FMA loop). v_permlane16_swap on loads 2p and 2p + 1 leaves in load 2p + s,
  // lane l: columns 8 (16 s + l % 16) .. +7 of row r + 4p + sigma(l / 16), sigma = (0, 2, 1, 3).
  // So lane l's B fragment for column 8 (16 s + l % 16) + j is half j of loads s, 2 + s, .., 14 + s,
  // K rows r + 4t + sigma(l / 16) for t = 0..7, and its A fragment holds the activations of those
  // rows; the 16 MFMAs (s, j) of a batch share the A fragment. Rows past the wavefront's range
  // have zero weights (their loads re-read its last row and are replaced by zeros) and zero
  // activations.
  bool fma_loop = true;
  if constexpr (MF) {
    static_assert(kRowsPerLoad == 2 && MM >= 2 && MM <= 8, "matrix-core form: 256-column strips, 2 <= M <= 8");
    const int g = lane >> 4, n16 = lane & 15;
    const int sig = g == 1 ? 2 : (g == 2 ? 1 : g);
    const int am = n16 & 7;       // the activation row of this lane's A fragment
    const bool alo = n16 >= 8;    // ... its lo parts (A rows 8-15)
    const int nb = (k1 - k0 + kMfBatch - 1) / kMfBatch;
    const bool col_ok = col < N;
    const _Float16* bp = B + min(col, N - 8);
    // 16 weight loads of the batch at row r: rows past the wavefront's range re-read its last row
    // (their values are replaced by zeros once they have landed)
    u32x4 w[16];
    auto load_batch = [&](int r) {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int row = r + 2 * u + sub;
        w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp + static_cast<size_t>(min(row, k1 - 1)) * N));
      }
    };
    float xr[kMfMaxBatches][8];
    float amax = 0.f;
    if (nb <= kMfMaxBatches && rows_per_wave >= kMfBatch) {
      // The first batch's weights stream while the activations come in (a wavefront that falls
      // back to the FMA loop drops them). Every activation this lane's A fragments need is then
      // loaded: rows past the wavefront's range (and rows am >= M) are 0.
      load_batch(k0);
#pragma unroll
      for (int bt = 0; bt < kMfMaxBatches; ++bt)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int row = k0 + kMfBatch * bt + 4 * t + sig;
          xr[bt][t] = (bt < nb && am < MM && row < k1) ? x_at(A, static_cast<size_t>(am) * K + row) : 0.f;
        }
      // |x| of row am over the wavefront's rows (the 4 lanes of each row combined); an inf or NaN
      // sends the wavefront to the FMA loop
      bool bad = false;
#pragma unroll
      for (int bt = 0; bt < kMfMaxBatches; ++bt)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float v = fabsf(xr[bt][t]);
          bad = bad || !(v <= 3.402823466e38f);
          amax = fmaxf(amax, v);
        }
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      fma_loop = __any(bad);
    }
    if (!fma_loop) {
      const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) - 15 : 0;  // amax * 2^-e in [2^14, 2^15)
      float4v acc2[2][8];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc2[s][j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int bt = 0; bt < kMfMaxBatches; ++bt) {
        if (bt >= nb) break;
        const int r = k0 + kMfBatch * bt;
        if (bt > 0) load_batch(r);
#pragma unroll
        for (int u = 0; u < 16; ++u)
          if (!col_ok || r + 2 * u + sub >= k1) w[u] = u32x4{0u, 0u, 0u, 0u};
        half8 af;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          _Float16 hi, lo;
          split_hi_lo(__builtin_ldexpf(xr[bt][t], -e), hi, lo);
          af[t] = alo ? lo : hi;
        }
#pragma unroll
        for (int p = 0; p < 8; ++p)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const auto sw = __builtin_amdgcn_permlane16_swap(w[2 * p][d], w[2 * p + 1][d], false, false);
            w[2 * p][d] = sw[0];
            w[2 * p + 1][d] = sw[1];
          }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            half8 bf;
#pragma unroll
            for (int t = 0; t < 8; ++t) bf[t] = __builtin_bit_cast(half8, w[2 * t + s])[j];
            acc2[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc2[s][j], 0, 0, 0);
          }
      }
      // Lane l, register i of acc2[s][j]: A row 4 (l / 16) + i, column 8 (16 s + l % 16) + j, i.e. the
      // hi part of activation row m = 4 (l / 16 % 2) + i in lanes 0-31 and its lo part in lanes
      // 32-63. Each lane writes its 8 consecutive columns as two 16-byte writes, scaled back by
      // 2^e_m (lane m holds e_m): the hi parts into this wavefront's first partial row of the LDS
      // reduction, the lo parts into its second, which the reduction adds. (One 4-byte write per
      // value made 8-way bank conflicts: 9 us of a 26 us M = 8 launch.)
      const int mrow = 4 * (g & 1);
      int er[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) er[i] = __shfl(e, mrow + i);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (mrow + i >= MM) continue;
          float* dst = &red[kRowsPerLoad * wave + (g >> 1)][mrow + i][(16 * s + n16) * 8];
#pragma unroll
          for (int h = 0; h < 2; ++h)
            *reinterpret_cast<float4v*>(dst + 4 * h) =
                float4v{__builtin_ldexpf(acc2[s][4 * h][i], er[i]), __builtin_ldexpf(acc2[s][4 * h + 1][i], er[i]),
                        __builtin_ldexpf(acc2[s][4 * h + 2][i], er[i]), __builtin_ldexpf(acc2[s][4 * h + 3][i], er[i])};
        }
    }
  }
  if (fma_loop && col < N) {
    constexpr int U = S::loads;
    constexpr int RB = U * kRowsPerLoad;  // rows of a batch
    const _Float16* bp = B + col + static_cast<size_t>(sub) * N;
    int k = k0;
    for (; k + RB <= k1; k += RB) {
      u32x4 w[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        w[u] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(bp + static_cast<size_t>(k + u * kRowsPerLoad) * N));
      if constexpr (S::issue) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float a[MM];
        act(k + u * kRowsPerLoad, true, a);
        fma_row<MM>(acc, a, w[u]);
      }
    }
    if (k < k1) {
      // Last, partial batch: all U loads still go out together; rows past the slice re-read its
      // last row and are not used (skipped, not multiplied by zero, so inf/NaN weights cannot leak
      // in).
      u32x4 w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = min(k + u * kRowsPerLoad + sub, k1 - 1);
        w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(B + col + static_cast<size_t>(r) * N));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float a[MM];
        act(k + u * kRowsPerLoad, false, a);
        if (k + u * kRowsPerLoad + sub < k1) fma_row<MM>(acc, a, w[u]);
      }
    }
  }

  const int part_row = wave * kRowsPerLoad + sub;
  if constexpr (MM == 1) {
    // One column per thread (threads 0 .. kStripCols-1, whole wavefronts): the partial rows in
    // order, then (split K) the slices in slice order, with every partial load issued
    // unconditionally (a thread past N reads column N - 1 and stores nothing).
    static_assert(kStripCols % kWave == 0 && kStripCols <= kThreads, "whole wavefronts own the columns");
    *reinterpret_cast<float4v*>(&red[part_row][0][lcol]) = float4v{acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
    *reinterpret_cast<float4v*>(&red[part_row][0][lcol + 4]) = float4v{acc[0][4], acc[0][5], acc[0][6], acc[0][7]};
    __syncthreads();
    const int t = threadIdx.x;
    const bool owner = t < kStripCols;  // uniform per wavefront
    const int c = strip * kStripCols + t;
    const bool live = owner && c < N;
    float mine = 0.f;
    if (owner) {
      mine = red[0][0][t];
#pragma unroll
      for (int w = 1; w < kParts; ++w) mine += red[w][0][t];
    }
    if (ksplit == 1) {
      if (live) C[c] = mine + (bias != nullptr ? bias[c] : 0.f);
      return;
    }
    if (live) store_coherent(part + static_cast<size_t>(kpart) * N + c, mine);
    if (!arrive_last_coherent(counters + strip * kCounterStride, static_cast<uint32_t>(ksplit))) return;
    if (owner) {
      const float* pc = part + min(c, N - 1);
      constexpr int kZBatch = 16;
      float sum = 0.f;
      for (int z0 = 0; z0 < ksplit; z0 += kZBatch) {
        float v[kZBatch];
#pragma unroll
        for (int b = 0; b < kZBatch; ++b) v[b] = z0 + b < ksplit ? load_coherent(pc + static_cast<size_t>(z0 + b) * N) : 0.f;
#pragma unroll
        for (int b = 0; b < kZBatch; ++b)
          if (z0 + b < ksplit) sum += v[b];
      }
      if (live) C[c] = sum + (bias != nullptr ? bias[c] : 0.f);
    }
    reset_counter(counters + strip * kCounterStride);
    return;
  }

  // Partial rows -> LDS, then the strip's MM x kStripCols sums are handed out in groups of kGW
  // consecutive columns of one row (4 for M >= 4, so that the split reduction moves them with
  // 16-byte coherent accesses; single columns below that): group g is row g / (kStripCols / kGW),
  // columns strip*kStripCols + kGW*(g % (kStripCols / kGW)) .., summed over the partial rows in
  // order. Every row of A goes through LDS in the same round, so one barrier serves all of them.
  if (fma_loop) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      *reinterpret_cast<float4v*>(&red[part_row][m][lcol]) = float4v{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
      *reinterpret_cast<float4v*>(&red[part_row][m][lcol + 4]) = float4v{acc[m][4], acc[m][5], acc[m][6], acc[m][7]};
    }
  }
  __syncthreads();
  constexpr int kGW = MM >= 4 ? 4 : 1;
  using V = std::conditional_t<kGW == 4, float4v, float>;
  constexpr int kRowGroups = kStripCols / kGW;
  constexpr int kGroups = MM * kRowGroups;
  constexpr int kGroupsPerThread = (kGroups + kThreads - 1) / kThreads;
  const int t = threadIdx.x;
  // groups that do not fill the last round cover only part of the threads
  auto group_in = [&](int i) { return kGroups % kThreads == 0 || t + i * kThreads < kGroups; };
  auto group_row = [&](int i) { return (t + i * kThreads) / kRowGroups; };
  auto group_col = [&](int i) { return strip * kStripCols + ((t + i * kThreads) % kRowGroups) * kGW; };
  auto group_live = [&](int i) { return group_in(i) && group_col(i) < N; };  // N % 8 == 0: whole groups
  auto lds_at = [&](int w, int i) {
    const float* p = &red[w][group_row(i)][group_col(i) - strip * kStripCols];
    if constexpr (kGW == 4) return *reinterpret_cast<const float4v*>(p);
    else return *p;
  };
  V mine[kGroupsPerThread];
#pragma unroll
  for (int i = 0; i < kGroupsPerThread; ++i) {
    mine[i] = V{};
    if (group_in(i)) {
      V s = lds_at(0, i);
#pragma unroll
      for (int w = 1; w < kParts; ++w) s += lds_at(w, i);
      mine[i] = s;
    }
  }
  auto store_out = [&](int i, V v) {
    const int c = group_col(i);
    float* o = C + static_cast<size_t>(group_row(i)) * N + c;
    if constexpr (kGW == 4) {
      if (bias != nullptr) v += float4v{bias[c], bias[c + 1], bias[c + 2], bias[c + 3]};
      *reinterpret_cast<float4v*>(o) = v;
    } else {
      *o = v + (bias != nullptr ? bias[c] : 0.f);
    }
  };

  if (ksplit == 1) {
#pragma unroll
    for (int i = 0; i < kGroupsPerThread; ++i)
      if (group_live(i)) store_out(i, mine[i]);
    return;
  }

  // slice z's partial of group i sits at float offset (z * MM + row) * N + col of the workspace
  const __amdgpu_buffer_rsrc_t slices = coherent_rsrc(part, static_cast<uint32_t>(ksplit) * MM * N * 4u);
  auto slot = [&](int z, int i) { return (static_cast<size_t>(z) * MM + group_row(i)) * N + group_col(i); };
  auto publish = [&](int i, V v) {
    if constexpr (kGW == 4) store_coherent4(slices, static_cast<uint32_t>(slot(kpart, i) * 4u), v);
    else store_coherent(part + slot(kpart, i), v);
  };
  auto fetch = [&](int z, int i) -> V {
    // with Sched::uncond, a group that is not live (past N, or past the M rows for M = 5..7) reads
    // the strip's first slot of slice z instead and its value is dropped
    const size_t sl = !S::uncond || group_live(i) ? slot(z, i)
                                                           : static_cast<size_t>(z) * MM * N + strip * kStripCols;
    if constexpr (kGW == 4) return load_coherent4(slices, static_cast<uint32_t>(sl * 4u));
    else return load_coherent(part + sl);
  };
#pragma unroll
  for (int i = 0; i < kGroupsPerThread; ++i)
    if (group_live(i)) publish(i, mine[i]);
  if (!arrive_last_coherent(counters + strip * kCounterStride, static_cast<uint32_t>(ksplit))) return;
  // Slices are added in slice order; loads are issued kZBatch slices at a time (for all of the
  // thread's groups) so their latencies overlap. Every slice, this one's included, is read back
  // from the workspace. Sixteen at a time covers the 16 slices of a 4096-row K in one round trip
  // (graph-timed, 4096^2: M = 4 10.31 -> 10.02 us, M = 8 13.08 -> 12.93 against 8 at a time). The
  // batch holds at most 16 loads per thread (64 registers with float4 groups): a thread with two
  // groups (512-column strips at M = 8) takes 8 slices per round trip.
  constexpr int kZBatch = kGroupsPerThread > 1 ? (16 / kGroupsPerThread > 0 ? 16 / kGroupsPerThread : 1) : 16;
  V s[kGroupsPerThread];
#pragma unroll
  for (int i = 0; i < kGroupsPerThread; ++i) s[i] = V{};
  for (int z0 = 0; z0 < ksplit; z0 += kZBatch) {
    V v[kZBatch][kGroupsPerThread];
#pragma unroll
    for (int b = 0; b < kZBatch; ++b)
#pragma unroll
      for (int i = 0; i < kGroupsPerThread; ++i)
        v[b][i] = (z0 + b < ksplit && (S::uncond || group_live(i))) ? fetch(z0 + b, i) : V{};
#pragma unroll
    for (int b = 0; b < kZBatch; ++b)
#pragma unroll
      for (int i = 0; i < kGroupsPerThread; ++i)
        if (z0 + b < ksplit) s[i] += v[b][i];
  }
#pragma unroll
  for (int i = 0; i < kGroupsPerThread; ++i)
    if (group_live(i)) store_out(i, s[i]);
  reset_counter(counters + strip * kCounterStride);
}

struct Split {
  int ksplit;         // slices actually launched
  int rows_per_wave;  // K rows per wavefront (a slice is kWaves times that)
};

Split split_for(int K, int ksplit) {
  if (K <= 0) return {1, 0};
  if (ksplit < 1) ksplit = 1;
  const int rpw = ceil_div(ceil_div(K, ksplit), kWaves);
  return {ceil_div(K, rpw * kWaves), rpw};
}

template <typename TX>
using SkinnyFn = void (*)(const TX*, const _Float16*, float*, const float*, float*, uint32_t*, int, int, int, int, int);

// The schedule of each M and strip width: graph-timed sweeps on MI355X of 2-16 loads per batch,
// with and without the issue barrier, over M = 1..8 and K x N in {4096^2, 1024 x 3072,
// 14336 x 4096, 1024^2} (256-column strips) and {4096 x 14336, 4096 x 11008} (512), weights
// rotated past the Infinity Cache; each entry is the best sum over its shapes (the runner-up is
// within 1-2 %). The partial-sum loads of M >= 4 are unconditional except for M = 6 and 8.
template <int MM, int COLS>
struct SchedFor;
template <int MM> struct SchedFor<MM, 256> {
  static constexpr int loads = MM == 1 || MM == 4 || MM == 8 ? 4 : 8;
  static constexpr bool issue = MM >= 5;
  using type = Sched<256, loads, issue, MM >= 4 && MM != 6 && MM != 8>;
};
template <int MM> struct SchedFor<MM, 512> {
  static constexpr int loads = MM == 2 || MM == 3 || MM == 7 || MM == 8 ? 16 : 8;
  static constexpr bool issue = !(MM >= 4 && MM <= 6);
  using type = Sched<512, loads, issue, MM >= 4 && MM != 6 && MM != 8>;
};

// Strip width: 256 columns up to N = 8192, 512 above. With few strips the split is deep and the
// last arriver's read-back (slices x M x strip width) dominates the exchange, which the narrow
// strips cut 4x (1 x 4096^2: 9.16 -> 8.63 us; 6 x 4096^2: 14.87 -> 10.98); with many strips the
// split is shallow already and the 1 KB rows stream slightly better (1 x 4096 x 11008: 16.77 us
// with 512 columns, 16.90 with 256; 8 x 4096 x 14336: 27.3 vs 31.9).
int strip_cols(int M, int N) {
  (void)M;
  return N <= 8192 ? 256 : 512;
}

template <typename TX, int COLS>
SkinnyFn<TX> skinny_fn_w(int M) {
  switch (M) {
    case 1: return skinny_kernel<TX, 1, typename SchedFor<1, COLS>::type>;
    case 2: return skinny_kernel<TX, 2, typename SchedFor<2, COLS>::type>;
    case 3: return skinny_kernel<TX, 3, typename SchedFor<3, COLS>::type>;
    case 4: return skinny_kernel<TX, 4, typename SchedFor<4, COLS>::type>;
    case 5: return skinny_kernel<TX, 5, typename SchedFor<5, COLS>::type>;
    case 6: return skinny_kernel<TX, 6, typename SchedFor<6, COLS>::type>;
    case 7: return skinny_kernel<TX, 7, typename SchedFor<7, COLS>::type>;
    default: return skinny_kernel<TX, 8, typename SchedFor<8, COLS>::type>;
  }
}
// The matrix-core form (skinny_kernel's MF) runs where it pays: M = 8 on 256-column strips with
// 32..128 K rows per wavefront. Graph-timed against the FMA loop, weights rotated past the
// Infinity Cache, us (K x N): 4096 x 4096 12.69 vs 12.95, 11008 x 4096 20.50 vs 25.52, 14336 x 4096
// 24.80 vs 29.29, 4096 x 8192 16.52 vs 19.18. Smaller M lose: one batch per wavefront leaves the
// matrix-core work and the hi/lo split exposed next to the FMAs they replace (M = 7, 4096^2:
// 12.62 vs 11.24; M = 2..6: 1.5-3 us slower); so do wavefronts with fewer rows than a batch.
bool use_mf(int M, int cols, int rows_per_wave) {
  return M == 8 && cols == 256 && rows_per_wave >= kMfBatch && rows_per_wave <= kMfBatch * kMfMaxBatches;
}
template <typename TX>
SkinnyFn<TX> skinny_fn(int M, int cols, bool mf) {
  if (mf) return skinny_kernel<TX, 8, typename SchedFor<8, 256>::type, true>;
  return cols == 256 ? skinny_fn_w<TX, 256>(M) : skinny_fn_w<TX, 512>(M);
}

size_t workspace_bytes(int M, int N, int ksplit) {
  if (ksplit <= 1 || M <= 0 || N <= 0) return 0;
  return static_cast<size_t>(ksplit) * M * N * sizeof(float);
}

size_t counters_needed(int M, int N, int ksplit) {
  if (ksplit <= 1 || M <= 0 || N <= 0) return 0;
  return counter_bytes(static_cast<size_t>(ceil_div(N, strip_cols(M, N))));
}

// Up to one 8-wavefront workgroup per CU, rounded down so that no workgroups are left for a second
// round (1 x 4096 x 14336 on 512-column strips: 280 workgroups 28.9 us, 224 workgroups 21.9 us),
// each wavefront streaming >= min_rows rows; then, within a factor of two below that, a split that
// gives every wavefront whole blocks of kPlanBlockRows rows (1 x 4096 x 12288: 8 slices 18.5 us,
// 10 slices 19.8 us). Chosen from graph-timed sweeps over M = 1..8 and K x N in {4096^2,
// 4096 x 11008, 4096 x 14336, 11008 x 4096}, weights rotated past the Infinity Cache.
int plan_with(int M, int N, int K, int num_cus, int cols) {
  if (N <= 0 || K <= 0 || num_cus <= 0) return 1;
  const int nstrips = ceil_div(N, cols);
  int ks = num_cus / nstrips;
  // M = 1 keeps a full 16-row block per wavefront (6.3 vs 7.2 us at 1x1024x3072); larger M gain
  // more from the extra slices than they lose to a partial block (10.8 vs 11.3 us at 4x1024x3072).
  const int min_rows = M == 1 ? 16 : kMinRows;
  const int cap = K / (kWaves * min_rows) > 1 ? K / (kWaves * min_rows) : 1;
  ks = ks < 1 ? 1 : (ks > cap ? cap : ks);
  for (int d = ks; d >= 1 && 2 * d >= ks; --d) {
    if (K % (kWaves * kPlanBlockRows * d) == 0) {
      ks = d;
      break;
    }
  }
  return split_for(K, ks).ksplit;
}

template <typename TX>
int skinny_launch(const TX* A, const uint16_t* B, float* C, const float* bias, int M, int N, int K, int ksplit,
                  void* ws, size_t ws_bytes, uint32_t* counters_in, size_t counter_bytes_in, void* stream) {
  if (M < 0 || N < 0 || K < 0 || M > G16_SKINNY_MAX_M || K % 8 != 0 || N % 8 != 0) return G16_E_SHAPE;
  if (M == 0 || N == 0) return G16_OK;
  if (ksplit < 1 || ksplit > 4096) return G16_E_SPLIT;
  if (C == nullptr || (K > 0 && (A == nullptr || B == nullptr))) return G16_E_NULL;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return G16_E_ALIGN;
  const Split sp = split_for(K, ksplit);
  // the split partials are addressed through one buffer descriptor: 32-bit byte offsets
  if (workspace_bytes(M, N, sp.ksplit) > 0x7fffffffu) return G16_E_SPLIT;
  const int cols = strip_cols(M, N);
  const int nstrips = ceil_div(N, cols);
  float* part = nullptr;
  uint32_t* counters = nullptr;
  if (sp.ksplit > 1) {
    if (ws == nullptr || ws_bytes < workspace_bytes(M, N, sp.ksplit)) return G16_E_WORKSPACE;
    if (counters_in == nullptr || counter_bytes_in < counters_needed(M, N, sp.ksplit)) return G16_E_WORKSPACE;
    if (!aligned16(ws) || !aligned16(counters_in)) return G16_E_ALIGN;
    counters = counters_in;
    part = static_cast<float*>(ws);
  }
  const dim3 grid(static_cast<unsigned>(nstrips) * static_cast<unsigned>(sp.ksplit)), block(kThreads);
  return launch(skinny_fn<TX>(M, cols, use_mf(M, cols, sp.rows_per_wave)), grid, block, static_cast<hipStream_t>(stream), A,
                reinterpret_cast<const _Float16*>(B), C, bias, part, counters, N, K, sp.rows_per_wave, sp.ksplit,
                nstrips);
}

__global__ void clear_words(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of `scratch` on the current device, looked up once per device with that device
// current. *fresh is set on the call that did the lookup (the counters then need their first
// clear). Returns nullptr (and the HIP status in *err) when the lookup fails.
unsigned char* scratch_on_current_device(int* err, bool* fresh) {
  static std::mutex mu;
  static void* ptr[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    *err = static_cast<int>(hipErrorInvalidDevice);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  *fresh = false;
  if (ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *err = static_cast<int>(e != hipSuccess ? e : hipErrorInvalidSymbol);
      return nullptr;
    }
    ptr[dev] = p;
    *fresh = true;
  }
  return static_cast<unsigned char*>(ptr[dev]);
}

}  // namespace
}  // namespace g16

extern "C" int g16_skinny_f32in_noalloc(const float* A, const uint16_t* B, float* C, const float* bias, int M,
                                        int N, int K, int ksplit, void* stream) {
  // Sizes are checked before any HIP call: the split must fit the static scratch.
  if (M < 0 || N < 0 || K < 0 || M > G16_SKINNY_MAX_M || K % 8 != 0 || N % 8 != 0) return G16_E_SHAPE;
  if (M == 0 || N == 0) return G16_OK;
  if (ksplit < 1 || ksplit > 4096) return G16_E_SPLIT;
  const g16::Split sp = g16::split_for(K, ksplit);
  if (g16::workspace_bytes(M, N, sp.ksplit) > G16_NOALLOC_PARTIAL_BYTES ||
      g16::counters_needed(M, N, sp.ksplit) > G16_NOALLOC_COUNTER_BYTES)
    return G16_E_TOO_LARGE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  g16::StreamDeviceScope on_stream_device(st);  // the stream's device is current for the lookup
  int err = 0;
  bool fresh = false;
  unsigned char* base = g16::scratch_on_current_device(&err, &fresh);
  if (base == nullptr) return err;
  auto* counters = reinterpret_cast<uint32_t*>(base);
  if (fresh) {
    // First use on this device: zero the counters with a kernel (not a memset node, so a caller
    // capturing this call into a graph replays a plain kernel); every later call leaves them zero.
    constexpr int kWords = G16_NOALLOC_COUNTER_BYTES / 4;
    const int rc = g16::launch(g16::clear_words, dim3((kWords + 255) / 256), dim3(256), st, counters, kWords);
    if (rc != 0) return rc;
  }
  return g16::skinny_launch<float>(A, B, C, bias, M, N, K, ksplit, base + G16_NOALLOC_COUNTER_BYTES,
                                   G16_NOALLOC_PARTIAL_BYTES, counters, G16_NOALLOC_COUNTER_BYTES, stream);
}

extern "C" int g16_skinny_plan(int M, int N, int K, int num_cus) {
  return g16::plan_with(M, N, K, num_cus, g16::strip_cols(M, N));
}

extern "C" int g16_skinny_strip_cols(int M, int N) { return g16::strip_cols(M, N); }

extern "C" size_t g16_skinny_workspace_bytes(int M, int N, int K, int ksplit) {
  if (K <= 0) return 0;
  return g16::workspace_bytes(M, N, g16::split_for(K, ksplit).ksplit);
}

extern "C" size_t g16_skinny_counter_bytes(int M, int N, int K, int ksplit) {
  if (K <= 0) return 0;
  return g16::counters_needed(M, N, g16::split_for(K, ksplit).ksplit);
}

extern "C" int g16_skinny_f32in(const float* A, const uint16_t* B, float* C, const float* bias, int M, int N, int K,
                                int ksplit, void* workspace, size_t workspace_bytes, uint32_t* counters,
                                size_t counter_bytes, void* stream) {
  return g16::skinny_launch<float>(A, B, C, bias, M, N, K, ksplit, workspace, workspace_bytes, counters, counter_bytes,
                                   stream);
}

extern "C" int g16_skinny_f16in(const uint16_t* A, const uint16_t* B, float* C, const float* bias, int M, int N,
                                int K, int ksplit, void* workspace, size_t workspace_bytes, uint32_t* counters,
                                size_t counter_bytes, void* stream) {
  return g16::skinny_launch<_Float16>(reinterpret_cast<const _Float16*>(A), B, C, bias, M, N, K, ksplit, workspace,
                                      workspace_bytes, counters, counter_bytes, stream);
}
