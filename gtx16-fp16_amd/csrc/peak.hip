// Instruction and bandwidth peaks of the part the kernels run on: the MI355X counterpart of the
// reference's bench/peak.py:1-63 (FFMA / HFMA2 / mma.sync on Turing). It calibrates the
// denominators the benchmark's rooflines use, under the clocks the part actually holds.
//
//   kind 0: fp32 FMA on the VALU (v_fma_f32), 8 independent chains per lane;
//   kind 1: packed fp16 FMA (v_pk_fma_f16), 8 chains of half2 per lane;
//   kind 2: v_mfma_f32_32x32x16_f16, 8 independent accumulators per wavefront;
//   kind 3: v_mfma_f32_16x16x32_f16, 16 independent accumulators per wavefront;
//   kinds 4, 5: kinds 2, 3 with operands of random fp16 bit patterns instead of the near-constant
//           ones of kinds 2, 3. The MFMA datapath's power depends on how many operand bits toggle,
//           and the part lowers its clock to hold its power limit, so these give the rate a GEMM
//           on real data can reach; 2 and 3 give the rate at the part's top clock.
//   kind 6: LDS reads, ds_read_b128 (16 bytes per lane), 8 in flight per wavefront;
//   kind 7: LDS transposing reads, ds_read_b64_tr_b16 (8 bytes per lane), 8 in flight;
//           kinds 6 and 7 give the LDS read bandwidth a CU sustains for the two fragment reads
//           the GEMM issues (A fragments are 16-byte reads, B fragments transposing reads);
//   kind 8 (g16_peak_mfma_data): the 256x256 GEMM tile's own MFMA stream without its memory
//           traffic. Each wavefront runs the per-step work of one of that tile's wavefronts: 8 A
//           and 4 B fragments, 32 v_mfma_f32_16x16x32_f16 into 32 accumulators in the tile's
//           snake order (consecutive MFMAs share one operand, and every MFMA changes the other),
//           on operand values the caller supplies (the benchmark passes fp16 of N(0,1) for A and
//           of N(0, 0.02^2) for B, the distributions of its 4096^3 workload), two fragment sets
//           alternating step by step as the tile's K steps do. Its rate is the ceiling the GEMM's
//           MFMA stream meets on that data under the part's power limit.
// and a streaming read of a large buffer (16-byte loads, grid-stride) for HBM bandwidth.
// Everything stays in registers except the read stream; results are folded into `out` so the
// compiler cannot drop the work. Workgroup 0's first wavefront can also report the shader clock
// cycles and the 100 MHz reference ticks its loop took (s_memtime, s_memrealtime), which give the
// clock the part held.
#include "g16_common.hpp"

namespace g16 {
namespace {

typedef _Float16 half2x __attribute__((ext_vector_type(2)));

// Loop clock of workgroup 0, wavefront 0: {shader cycles, 100 MHz reference ticks} -> clk[0..1].
struct LoopClock {
  unsigned long long c0 = 0, r0 = 0;
  __device__ void start() {
    c0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  __device__ void stop(unsigned long long* clk) const {
    const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (clk != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
      clk[0] = c1 - c0;
      clk[1] = r1 - r0;
    }
  }
};

// Random fp16 bit pattern: random sign and 10 mantissa bits, exponent in [2^-3, 2^0) so that
// 20000 accumulations of 16-term products stay far from overflow.
__device__ inline _Float16 random_half(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  const uint16_t bits = static_cast<uint16_t>((x & 0x83ffu) | ((12u + ((x >> 10) & 3u)) << 10));
  return __builtin_bit_cast(_Float16, bits);
}

__global__ __launch_bounds__(256) void peak_ffma(float* out, unsigned long long* clk, float a, float b, int iters) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(threadIdx.x + i);
  LoopClock lc;
  lc.start();
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = fmaf(x[i], a, b);
  lc.stop(clk);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void peak_hfma2(float* out, unsigned long long* clk, float af, float bf, int iters) {
  const half2x a = {static_cast<_Float16>(af), static_cast<_Float16>(af)};
  const half2x b = {static_cast<_Float16>(bf), static_cast<_Float16>(bf)};
  half2x x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 v = static_cast<_Float16>((threadIdx.x + i) * 1e-3f);
    x[i] = half2x{v, v};
  }
  LoopClock lc;
  lc.start();
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = x[i] * a + b;
  lc.stop(clk);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += static_cast<float>(x[i].x) + static_cast<float>(x[i].y);
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// MFMA operands: near-constant (a depends on the lane, b on the element only) or random bits
template <bool RANDOM>
__device__ inline void mfma_operands(half8& a, half8& b, float seed) {
  const uint32_t g = (blockIdx.x * blockDim.x + threadIdx.x) * 16u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = RANDOM ? random_half(g + i) : static_cast<_Float16>(seed * (threadIdx.x + i));
    b[i] = RANDOM ? random_half(g + 8 + i) : static_cast<_Float16>(seed * i);
  }
}

template <bool RANDOM>
__global__ __launch_bounds__(256) void peak_mfma32(float* out, unsigned long long* clk, float seed, int iters) {
  float16v acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = float16v{};
  half8 a, b;
  mfma_operands<RANDOM>(a, b, seed);
  LoopClock lc;
  lc.start();
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[i], 0, 0, 0);
  lc.stop(clk);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][threadIdx.x & 15];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <bool RANDOM>
__global__ __launch_bounds__(256) void peak_mfma16(float* out, unsigned long long* clk, float seed, int iters) {
  float4v acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = float4v{0.f, 0.f, 0.f, 0.f};
  half8 a, b;
  mfma_operands<RANDOM>(a, b, seed);
  LoopClock lc;
  lc.start();
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[i], 0, 0, 0);
  lc.stop(clk);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += acc[i][threadIdx.x & 3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Kind 8: per lane, fragment f (0-7: A_f, 8-11: B_(f-8)) of set s is the 8 halves at
// ops[(((blockIdx.x % ngroups) * 256 + threadIdx.x) * 2 + s) * 12 + f], so with ngroups = the
// grid every wavefront has operands of its own (the two that share a SIMD included). One iteration
// is two steps (set 0, set 1)
// of 32 MFMAs; m = 4 i + jj multiplies A_i by B_j, j = jj on even i and 3 - jj on odd i (the
// tile's order). All 32 accumulators (4 floats each) are stored: lane t of workgroup b writes
// out[(b * 256 + t) * 128 + (4 i + j) * 4 + r] = acc[i][j][r], the MFMA's register r of block
// (i, j): row 4 * (lane / 16) + r, column lane % 16 of the 16 x 16 block.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void peak_mfma_gemm_order(
    const half8* __restrict__ ops, int ngroups, float* __restrict__ out, unsigned long long* clk, int iters) {
  const half8* mine = ops + ((blockIdx.x % static_cast<unsigned>(ngroups)) * 256u + threadIdx.x) * 24u;
  half8 a[2][8], b[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) a[s][i] = mine[s * 12 + i];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[s][j] = mine[s * 12 + 8 + j];
  }
  float4v acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};
  LoopClock lc;
  lc.start();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int m = 0; m < 32; ++m) {
        const int i = m / 4, jj = m % 4, j = (i & 1) ? 3 - jj : jj;
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s][i], b[s][j], acc[i][j], 0, 0, 0);
      }
  }
  lc.stop(clk);
  float4v* o = reinterpret_cast<float4v*>(out + (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) * 128);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) o[4 * i + j] = acc[i][j];
}

// LDS read bandwidth: every wavefront reads 8 contiguous pieces of 64 lanes x W bytes (W = 16 for
// ds_read_b128, 8 for ds_read_b64_tr_b16; contiguous lanes touch distinct banks) from a 32 KB
// buffer, then waits for them; the reads are inline asm (volatile, with a memory clobber) so the
// compiler can neither drop, hoist nor merge them. Offsets stay inside the buffer: lane base
// < 256 * 16 = 4 KB and piece offsets d * 4 KB (d < 8), so the last byte read is below 32 KB.
// 32 KB per workgroup lets five workgroups (20 wavefronts) share a CU's 160 KB.
#define G16_LDS_READ8(INSN, V, A)                                                                  \
  asm volatile(INSN " %0, %8 offset:0\n\t" INSN " %1, %8 offset:4096\n\t" INSN " %2, %8 offset:8192\n\t" \
               INSN " %3, %8 offset:12288\n\t" INSN " %4, %8 offset:16384\n\t" INSN " %5, %8 offset:20480\n\t" \
               INSN " %6, %8 offset:24576\n\t" INSN " %7, %8 offset:28672\n\ts_waitcnt lgkmcnt(0)"    \
               : "=v"(V[0]), "=v"(V[1]), "=v"(V[2]), "=v"(V[3]), "=v"(V[4]), "=v"(V[5]), "=v"(V[6]),     \
                 "=v"(V[7])                                                                           \
               : "v"(A)                                                                               \
               : "memory")

template <bool TR>
__global__ __launch_bounds__(256) void peak_lds(float* out, unsigned long long* clk, float seed, int iters) {
  __shared__ u32x4 buf[2048];  // 32 KB
  for (int i = threadIdx.x; i < 2048; i += 256) {
    const uint32_t u = static_cast<uint32_t>(i) + static_cast<uint32_t>(seed);
    buf[i] = u32x4{u, u ^ 0x5555u, u * 3u, u * 7u};
  }
  __syncthreads();
  const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                            (__attribute__((address_space(3))) void*)&buf[0])) +
                        threadIdx.x * (TR ? 8u : 16u);
  uint32_t acc = 0;
  LoopClock lc;
  lc.start();
  for (int it = 0; it < iters; ++it) {
    if constexpr (TR) {
      u32x2 v[8];
      G16_LDS_READ8("ds_read_b64_tr_b16", v, base);
#pragma unroll
      for (int d = 0; d < 8; ++d) acc ^= v[d].x;
    } else {
      u32x4 v[8];
      G16_LDS_READ8("ds_read_b128", v, base);
#pragma unroll
      for (int d = 0; d < 8; ++d) acc ^= v[d].x;
    }
  }
  lc.stop(clk);
  out[blockIdx.x * blockDim.x + threadIdx.x] = static_cast<float>(acc & 0xffu);
}
#undef G16_LDS_READ8

// Grid-stride read of n16 16-byte chunks; every lane folds what it read into one float.
__global__ __launch_bounds__(256) void stream_read(const u32x4* __restrict__ p, size_t n16, float* out) {
  uint32_t acc = 0;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  constexpr int kDepth = 8;  // loads in flight per lane
  for (; i + (kDepth - 1) * stride < n16; i += kDepth * stride) {
    u32x4 v[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) v[d] = p[i + d * stride];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
  }
  for (; i < n16; i += stride) {
    const u32x4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = static_cast<float>(acc & 0xffu);
}

}  // namespace
}  // namespace g16

extern "C" double g16_peak_flops_per_lane_iter(int kind) {
  // work one lane contributes per loop iteration: flops for kinds 0-5 (MFMA: a wavefront's
  // flops / 64), LDS bytes read for kinds 6 and 7
  switch (kind) {
    case 0: return 8.0 * 2;                          // 8 fp32 FMAs
    case 1: return 8.0 * 2 * 2;                      // 8 packed fp16 FMAs
    case 2: case 4: return 8.0 * 32 * 32 * 16 * 2 / 64;      // 8 MFMA 32x32x16
    case 3: case 5: return 16.0 * 16 * 16 * 32 * 2 / 64;     // 16 MFMA 16x16x32
    case 6: return 8.0 * 16;                         // LDS bytes: 8 ds_read_b128
    case 7: return 8.0 * 8;                          // LDS bytes: 8 ds_read_b64_tr_b16
    case 8: return 64.0 * 16 * 16 * 32 * 2 / 64;     // two steps of 32 MFMA 16x16x32
    default: return 0.0;
  }
}

extern "C" int g16_peak_run_clocked(int kind, int blocks, int iters, float* out, unsigned long long* clocks,
                                    void* stream) {
  // out must hold blocks * 256 floats; clocks (may be NULL) receives 2 values
  if (blocks <= 0 || iters < 0) return G16_E_SHAPE;
  if (out == nullptr) return G16_E_NULL;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (kind) {
    case 0: return g16::launch(g16::peak_ffma, grid, block, s, out, clocks, 0.999f, 0.001f, iters);
    case 1: return g16::launch(g16::peak_hfma2, grid, block, s, out, clocks, 0.999f, 0.001f, iters);
    case 2: return g16::launch(g16::peak_mfma32<false>, grid, block, s, out, clocks, 1e-3f, iters);
    case 3: return g16::launch(g16::peak_mfma16<false>, grid, block, s, out, clocks, 1e-3f, iters);
    case 4: return g16::launch(g16::peak_mfma32<true>, grid, block, s, out, clocks, 1e-3f, iters);
    case 5: return g16::launch(g16::peak_mfma16<true>, grid, block, s, out, clocks, 1e-3f, iters);
    case 6: return g16::launch(g16::peak_lds<false>, grid, block, s, out, clocks, 1.0f, iters);
    case 7: return g16::launch(g16::peak_lds<true>, grid, block, s, out, clocks, 1.0f, iters);
    default: return G16_E_DTYPE;
  }
}

extern "C" int g16_peak_run(int kind, int blocks, int iters, float* out, void* stream) {
  return g16_peak_run_clocked(kind, blocks, iters, out, nullptr, stream);
}

extern "C" int g16_peak_mfma_data(int blocks, int iters, const uint16_t* operands, int ngroups, float* out,
                                  unsigned long long* clocks, void* stream) {
  // operands: ngroups * 256 * 24 fragments of 8 fp16 values; out: blocks * 256 * 128 floats
  if (blocks <= 0 || iters < 0 || ngroups <= 0) return G16_E_SHAPE;
  if (operands == nullptr || out == nullptr) return G16_E_NULL;
  if (!g16::aligned16(operands) || !g16::aligned16(out)) return G16_E_ALIGN;
  return g16::launch(g16::peak_mfma_gemm_order, dim3(static_cast<unsigned>(blocks)), dim3(256),
                     static_cast<hipStream_t>(stream), reinterpret_cast<const g16::half8*>(operands), ngroups, out,
                     clocks, iters);
}

extern "C" int g16_stream_read(const void* buf, size_t bytes, int blocks, float* out, void* stream) {
  // out must hold blocks * 256 floats; bytes must be a multiple of 16
  if (blocks <= 0 || bytes % 16 != 0) return G16_E_SHAPE;
  if (buf == nullptr || out == nullptr) return G16_E_NULL;
  if (!g16::aligned16(buf)) return G16_E_ALIGN;
  return g16::launch(g16::stream_read, dim3(static_cast<unsigned>(blocks)), dim3(256), static_cast<hipStream_t>(stream),
                     static_cast<const g16::u32x4*>(buf), bytes / 16, out);
}
