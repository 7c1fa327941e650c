// Tiled fp16 GEMM on the gfx950 matrix cores, fp32 accumulation, with an optional deterministic
// split over K.
//
// Semantics (reference: src/gtx16_fp16/kernels.py:35-151, ops.py:92-108):
//   C[M,N] = rscale[row] * (A[M,K] @ B[K,N]) + bias[N], cast to fp32 or fp16 (nearest-even),
// scale first, then bias, then cast (kernels.py:116-133). A is the fp16 output of the rowscale
// cast (K contiguous), B the fp16 weight w_t (N contiguous).
//
// Structure:
//   * A workgroup owns a BM x BN output tile; each wavefront owns a (BM/WGM) x (BN/WGN) sub-tile
//     made of MFMA blocks with fp32 accumulators. The large tiles are 256x256 and 256x128 with 8
//     wavefronts (two per SIMD) on 16x16 blocks of v_mfma_f32_16x16x32_f16; smaller tiles
//     (128x128, 64x128, 64x64, 32x128) use 4 wavefronts on 32x32 blocks of
//     v_mfma_f32_32x32x16_f16 and serve small and medium M and split-K. Both instructions have the
//     same peak rate; on random operands the 16x16x32 one
//     draws less power, and at 4096^3 the part is power-limited (it holds ~1.6 GHz, not 2.4), so
//     the large tile runs 4-6 % faster with it.
//   * K advances in steps of BK through a ring of NSTAGE LDS stages filled by DMA
//     (buffer_load_dwordx4 ... lds), so operand tiles never pass through registers. Lanes whose
//     16-byte chunk lies outside the matrix (ragged M, N, K or a split-K slice boundary) are given
//     an out-of-range buffer offset, which makes the DMA write zeros.
//   * The DMA writes 1 KB per wavefront instruction (lane i -> bytes 16i..16i+15), so the LDS
//     layout is chosen through which global chunk each lane fetches: A is stored [row][k], B
//     [k][n] like the weight, each with a 16-byte-chunk XOR swizzle (swz_a, swz_b) that keeps the
//     fragment reads free of bank conflicts.
//   * MFMA operands need K-contiguous runs per lane (8 halves). A fragments are one 16-byte LDS
//     read each. B fragments use the gfx950 transposing read ds_read_b64_tr_b16: within each
//     16-lane group, lane p receives element p%4 of the 8-byte pieces addressed by lanes p/4 + 4j
//     (j = 0..3), so pointing lane q at B[k0 + q/4][n0 + 4(q%4)] hands lane p the run
//     B[k0..k0+3][n0 + p]; two such reads give the 8-deep run one operand needs.
//   * Schedules: the 8-wavefront tile runs a ping-pong between the two wavefronts of each SIMD
//     (one issues a step's MFMAs while the other reads LDS and issues DMA, swapping at every
//     barrier); the 4-wavefront tiles interleave DMA, MFMAs and the next step's fragment reads
//     (fragments double-buffered in registers) with one barrier per step.
//   * Tiles are assigned XCD-aware: the hardware deals workgroups round-robin over the 8 XCDs, so
//     workgroup b is mapped to tile (b % 8) * (T / 8) + b / 8 when the T tiles are a multiple of 8
//     (and, for unsplit grids of any other count, to the same contiguous runs of T / 8 or T / 8 + 1
//     tiles per XCD), giving each XCD a contiguous run of tiles, which a grouped (GROUP_M rows at a
//     time) order turns into a compact 2-D block that shares A rows and B columns in that XCD's L2.
//     An unsplit 256-row grid with more tiles than CUs is persistent: one workgroup per CU (a
//     multiple of 8) walks tiles b, b + G, b + 2G, ... of the same sequence.
//   * Resident A (the unsplit 32x128 tile with K <= kResidentSteps * 64, mm_t's GEMM path in one
//     launch): the workgroup reads its 32 rows of the fp32/fp16 activations itself, computes each
//     row's scale (rowscale_math.hpp, the rowscale kernel's arithmetic) and writes the scaled fp16
//     rows into LDS as the stage images of every K step, which then stay resident; only B streams
//     through the ring. No fp16 copy of A goes to HBM and no separate rowscale launch runs.
//   * Speculative fp16 A (the 4-wavefront tiles with fp16 activations, mm_t's GEMM path in one
//     launch): a row whose |max| does not exceed the threshold has scale 1, and its rowscale cast is
//     the activation itself. So the GEMM streams x as A and tracks the largest |x| it multiplies
//     (from the A fragments). If no row of the tile exceeds the threshold, the result is the cast
//     path's, bit for bit. Otherwise the tile is computed again with its A fragments multiplied in
//     registers by the rows' factors 2^-e (an exact product rounded once, with fp16 denormals kept:
//     the rowscale cast's value): unsplit tiles right away, split tiles by the slice that arrives
//     last (every flagged slice marks the arrival count), which recomputes every slice in slice
//     order -- the same sums the split reduction adds.
//   * Split-K: slice z of tile t covers K range [z*kchunk, (z+1)*kchunk). Every slice stores its
//     fp32 accumulators to the workspace in the lanes' own register order (fully coalesced 16-byte
//     device-coherent stores); the last slice to arrive adds all slices in slice order and runs the
//     epilogue. Deterministic, and bias/scale/cast are fused (the reference prefills C with the bias
//     and adds with fp32 atomics, kernels.py:119-122, ops.py:54-62).
#include <atomic>
#include <mutex>
#include <type_traits>

#include "g16_common.hpp"
#include "rowscale_math.hpp"

namespace g16 {
namespace {

constexpr int kGroupM = 8;
constexpr int kSplitAlign = 64;  // split-K slices start on a multiple of every tile's K step
// The planner's rule (M <= 64) splits no K below this: two slices of 256 cost more than they save
// (graph-timed: 16 x 8192 x 512 (M x N x K) 6.0 us unsplit, 7.1 split twice; 48 x 2048 x 512 6.2
// vs 7.2); at K = 1024 four slices win (64 x 1024^2 7.7 -> 7.1).
constexpr int kMinSplitK = 1024;
constexpr uint32_t kOob = 0x80000000u;  // buffer offset past every descriptor's range: reads 0

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) short4v lds_short4v;

// LDS byte address -> LDS address-space pointer (the transpose-read builtin takes one).
__device__ inline lds_short4v* lds4_at(uint32_t addr) { return reinterpret_cast<lds_short4v*>(static_cast<uintptr_t>(addr)); }

// 16-byte DMA global -> LDS: lane i's chunk at buffer offset `off` lands at LDS byte lds + 16 i.
// Issued as inline asm so the compiler's wait-counter bookkeeping does not see an LDS write it
// cannot tell apart from the stage being read (it would wait for the DMA before every LDS
// read); the kernel waits for its DMA explicitly (vmcnt 0) before the barrier that publishes a
// stage. Vector memory returns in order, so the compiler's own vmcnt waits stay correct (they can
// only wait longer) with these loads in flight. M0 (the LDS base of the DMA) is set and consumed
// inside the same statement; clang warns that m0 is reserved, but these kernels contain no other
// reader of M0 (no LDS-direct, GWS or message instructions): in the generated assembly every
// `s_mov_b32 m0` is one of these statements, immediately followed by its DMA.
// `lds_addr` is the LDS byte address (see lds_base) of the 1 KB the instruction fills.
__device__ inline void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_addr, uint32_t off) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(off), "s"(rsrc)
               : "memory", "m0");
}

// LDS byte address of a __shared__ object, taken once per kernel: converting a generic pointer to
// the LDS address space costs a 64-bit add and a null test, too much to repeat for every DMA
// instruction of a loop that issues few other instructions.
__device__ inline uint32_t lds_base(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)p));
}

template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int NSTAGE_, bool MF16_ = false>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_, NSTAGE = NSTAGE_;
  static constexpr int WAVES = WGM * WGN;
  static constexpr int THREADS = WAVES * kWave;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;  // wavefront sub-tile
  // MFMA shape: v_mfma_f32_16x16x32_f16 (MF16) or v_mfma_f32_32x32x16_f16. Same flops per cycle;
  // on random operands the 16x16x32 form draws less power, so a power-limited part holds a higher
  // clock with it (measured: +3 to +8 % per GEMM step at the same LDS traffic).
  static constexpr bool MF16 = MF16_;
  static constexpr int MB = MF16 ? 16 : 32;               // MFMA output block edge
  static constexpr int MK = MF16 ? 32 : 16;               // MFMA K depth
  static constexpr int TM = WTM / MB, TN = WTN / MB;      // MFMA blocks per wavefront
  static_assert(TM >= 1 && TN >= 1 && WTM % MB == 0 && WTN % MB == 0, "whole MFMA blocks");
  static_assert(!MF16 || (TM % 2 == 0 && TN % 2 == 0), "the epilogue stores 2x2 groups of 16x16 blocks");
  static_assert(BK == 32 || BK == 64, "K step");
  static constexpr int A_BYTES = BM * BK * 2;            // one stage of A
  static constexpr int B_BYTES = BK * BN * 2;            // one stage of B
  static constexpr int A_ROW_CHUNKS = BK / 8;            // 16-byte chunks per A row
  static constexpr int A_ROWS_PER_INSTR = 64 / A_ROW_CHUNKS;
  static constexpr int A_INSTR = A_BYTES / 1024 / WAVES;  // 1 KB DMA instructions per wavefront
  static constexpr int B_ROW_CHUNKS = BN / 8;            // 16-byte chunks per B row
  static constexpr int B_ROWS_PER_INSTR = 64 / B_ROW_CHUNKS;
  static constexpr int B_INSTR = B_BYTES / 1024 / WAVES;
  static_assert(A_INSTR >= 1 && B_INSTR >= 1 && A_BYTES % (1024 * WAVES) == 0 && B_BYTES % (1024 * WAVES) == 0,
                "every wavefront issues the same number of DMA instructions");
  static_assert(B_ROW_CHUNKS >= 8 && B_ROW_CHUNKS <= 64, "B swizzle needs >= 8 chunks per row");
  static constexpr int DMA_PER_STEP = A_INSTR + B_INSTR;  // per wavefront
  static_assert(NSTAGE >= 3 && (NSTAGE - 2) * DMA_PER_STEP <= 63, "vmcnt range");
  static_assert(!MF16 || A_ROW_CHUNKS == 4, "the 16x16x32 tile's A stage is the packed image");

  // LDS chunk swizzles (the LDS has 64 four-byte banks: a 256-byte period). Which lanes one LDS
  // cycle serves is not a plain run of consecutive lanes, so the forms below were chosen by
  // measuring read patterns on the part (cycles per read instruction with the LDS saturated):
  //   A (and the packed B^T): row r keeps chunk c at c ^ swz_a(r). 32x32 fragments (lane l: row
  //   l % 32, chunk l / 32): (r / (16 / RC)) % RC. 16x16x32 fragments (lane l: row l % 16, chunk
  //   l / 16): (r / 2) % 4, the packed layout's swizzle; (r / 4) % 4 doubled their read time.
  //   B (row-major, transposing reads; a 32-lane half reads 16 columns of 8 k rows): row k keeps
  //   chunk c at c ^ swz_b(k). With 128 columns (32x32 blocks), 4 * (k % 4); with 256 columns and
  //   16x16x32 blocks (k rows 0-3 and 8-11 in one half), 2 * (k % 4 + 4 * ((k / 8) % 2)), which
  //   puts the 8 rows' 32-byte pieces on 8 distinct bank ranges (4 * (k % 4) paired rows k and
  //   k + 8: 1.7x the read time). With 64 columns (128-byte rows, two to a bank period),
  //   4 * ((k / 2) % 2) + 2 * ((k / 8) % 2): rows k and k + 2 of one bank half take different
  //   64-byte ranges, and rows k and k + 8 different 32-byte pieces within them, so the 32x32 reads
  //   are conflict-free whichever of those row sets one LDS cycle serves. Every form gives every k
  //   row a lane reads in one step (k, k + 4, and k + MK on later substeps) the same swizzle.
  __device__ static int swz_a(int row) {
    if constexpr (MF16) return pack_swz(row);
    else return (row / (16 / A_ROW_CHUNKS)) % A_ROW_CHUNKS;
  }
  __device__ static int swz_b(int k) {
    if constexpr (MF16) return ((k & 3) + 4 * ((k >> 3) & 1)) << 1;
    else if constexpr (B_ROW_CHUNKS == 8) return (((k >> 1) & 1) << 2) | (((k >> 3) & 1) << 1);
    else return (k & 3) << 2;
  }
};

// K steps the resident-A tile keeps in LDS: 20 x 4 KB of A plus the 64 KB B ring (K <= 1280).
constexpr int kResidentSteps = 20;

using Cfg256 = TileCfg<256, 256, 32, 2, 4, 4, true>;  // 8 wavefronts (two per SIMD), 4-stage ring, 128 KB
using Cfg256n = TileCfg<256, 128, 32, 2, 4, 4, true>;  // the same schedule on half the columns, 96 KB
using Cfg128 = TileCfg<128, 128, 32, 2, 2, 4>;  // 64 KB: two workgroups per CU
using Cfg64 = TileCfg<64, 128, 64, 1, 4, 4>;
using Cfg32 = TileCfg<32, 128, 64, 1, 4, 4>;
using Cfg64x64 = TileCfg<64, 64, 64, 2, 2, 4>;  // 64 KB: the square 4-wavefront tile

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left alone: waits until at most N of this wavefront's
// vector-memory operations (here: the DMA of younger stages) are still in flight.
template <int N>
__device__ inline void wait_dma_le() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// s_waitcnt immediate for vmcnt(0) alone (expcnt 7, lgkmcnt 15 leave those counters alone), for
// __builtin_amdgcn_s_waitcnt, whose waits the compiler's own wait tracking takes into account.
constexpr int kWaitVmcnt0 = 0x0f70;
constexpr int kCpolNt = 2;  // cache policy bit nt of a buffer access: streaming (non-temporal)

// Shader-clock stamps of the latest GEMM launch: workgroup 0 of every launch records the shader
// cycles (s_memtime) and 100 MHz reference ticks (s_memrealtime) its main loop took, so
// 100 MHz * cycles / ticks is the clock the part held while that launch ran (the part is
// power-limited and its clock moves with load). g16_gemm_clock copies them out.
__device__ unsigned long long g_loop_clock[2];

// Largest of v over the 64 lanes, in every lane: DPP within each row of 16 lanes, then the four
// rows' results through scalar reads. (max is exact, so any order gives the rowscale kernel's
// value.)
__device__ inline float wave_max(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xb1>{}));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4e>{}));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// arrive_last_coherent with a value: every thread of the workgroup calls it after its coherent
// stores; the workgroup adds `add` to the counter and every thread gets the counter's value after
// that addition.
__device__ inline uint32_t arrive_add_coherent(uint32_t* counter, uint32_t add) {
  __shared__ uint32_t s_val;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed at the coherence point
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) s_val = __hip_atomic_fetch_add(counter, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
  __syncthreads();
  return s_val;
}
// Split counter of a speculative launch: the arrival count in the low kSpecShift bits, and bit
// kSpecShift + z set by slice z if its A exceeded the threshold (each slice adds its own bit once,
// so the fields never carry into each other).
constexpr int kSpecShift = 8;
constexpr int kSpecMaxSplit = 32 - kSpecShift;

// Workgroup barrier without the counter waits __syncthreads() adds: the caller has already waited
// for exactly the memory operations the next phase depends on. The memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ inline void phase_barrier() { asm volatile("s_barrier" ::: "memory"); }

// RESIDENT: A is unused; the kernel casts X (fp32 when x_f32, else fp16; threshold 2^texp) itself
// into resident LDS stages (the 32x128 tile, unsplit, K <= kResidentSteps * BK).
// SPEC: A is the fp16 activations, streamed as they are; tbits is the largest fp16 bit pattern
// not above the threshold 2^texp (texp >= -8, so every row exponent is <= 24). A tile with a larger
// |x| (or a NaN) is computed again with its A fragments rescaled in registers: unsplit, by the same
// workgroup; split, by the slice that arrives last, over every slice in slice order. A split
// slice that saw such a value publishes its rows' |max| in place of its partial tile. A tile that
// is computed again stores 1 into *spec_miss (when not NULL; pinned host memory).
template <class Cfg, bool OUT_F16, bool SPLITK, bool PACKED_A = false, bool PACKED_B = false, bool RESIDENT = false,
          bool SPEC = false>
__global__ __launch_bounds__(Cfg::THREADS) void hgemm_kernel(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                                                         void* __restrict__ Cv, const float* __restrict__ bias,
                                                         const float* __restrict__ rscale, float* __restrict__ part,
                                                         uint32_t* __restrict__ counters, int M, int N, int K,
                                                         int kchunk, int ksplit, int ntm, int ntn,
                                                         const void* __restrict__ X, int x_f32, int texp,
                                                         int tbits, uint32_t* __restrict__ spec_miss) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, TM = Cfg::TM, TN = Cfg::TN, MB = Cfg::MB, MK = Cfg::MK;
  constexpr int BK = Cfg::BK, NSTAGE = Cfg::NSTAGE;
  static_assert(!RESIDENT || (Cfg::BM == 32 && Cfg::BK == 64 && Cfg::WAVES == 4 && !SPLITK && !PACKED_A && !PACKED_B),
                "resident A: the unsplit 32x128 tile");
  static_assert(!SPEC || (Cfg::WAVES == 4 && !Cfg::MF16 && !PACKED_A && !PACKED_B && !RESIDENT),
                "speculative A: the 4-wavefront tiles, 32x32x16 blocks (lane l's A rows are l % 32)");
  constexpr int A_STAGES = RESIDENT ? kResidentSteps : NSTAGE;
  __shared__ __attribute__((aligned(1024))) unsigned char sA[A_STAGES][Cfg::A_BYTES];
  __shared__ __attribute__((aligned(1024))) unsigned char sB[NSTAGE][Cfg::B_BYTES];
  __shared__ float s_scale[(RESIDENT || SPEC) ? BM : 1];
  __shared__ float s_rowmax[SPEC ? BM : 1];  // speculative recomputation: the rows' |max|, then 2^-e
  const uint32_t sA_lds = lds_base(&sA[0][0]), sB_lds = lds_base(&sB[0][0]);

  // ---- tile assignment (XCD-aware, grouped) ----
  // Workgroups reach the 8 XCDs round-robin by linear index. Each XCD's workgroups get a contiguous
  // range of the grouped tile order below, so its L2 serves a compact block of tile rows and
  // columns: ranges of ntiles / 8 tiles; with an unsplit grid of another size, ranges of
  // floor(ntiles / 8) or one more. (For split grids of such sizes the linear order is kept: a
  // slice-major mapping measured 1-3 us slower there.)
  // A grid of fewer workgroups than tiles (the unsplit 256-row tiles past one round: one workgroup
  // per CU, a multiple of 8) is persistent: workgroup b computes tiles b, b + gridDim.x, ... in
  // turn, so each XCD still walks its own contiguous range, and no round of workgroups retires
  // and is dispatched again (65536 x 768 x 768 on 256 CUs: 101.9 -> 94.4 us; 65536 x 768 x 3072:
  // 371 -> 357 us). A split grid always has one workgroup per tile, so its early returns below
  // end the workgroup's only tile.
  const int ntiles = ntm * ntn;
  for (int work = blockIdx.x; work < ntiles; work += gridDim.x) {
    int lin = work;
    if (ntiles % 8 == 0) {
      lin = (lin % 8) * (ntiles / 8) + lin / 8;
    } else if (gridDim.y == 1) {
      const int xcd = lin % 8, q8 = ntiles / 8, r8 = ntiles % 8;
      lin = xcd * q8 + min(xcd, r8) + lin / 8;  // XCD x holds q8 + (x < r8) workgroups
    }
    const int per_group = kGroupM * ntn;
    const int first_m = (lin / per_group) * kGroupM;
    const int gsz = min(ntm - first_m, kGroupM);
    const int tm = first_m + (lin % per_group) % gsz;
    const int tn = (lin % per_group) / gsz;
    const int tile = tm * ntn + tn;
    const int m0 = tm * BM, n0 = tn * BN;
    const int z = blockIdx.y;
    // this slice's K range (the speculative path's recomputation walks every slice's range)
    int kbeg = z * kchunk;
    int kend = min(K, kbeg + kchunk);
    int nk = kend > kbeg ? ceil_div(kend - kbeg, BK) : 0;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool stamps = blockIdx.x == 0 && blockIdx.y == 0;  // workgroup 0 records the loop's clock
    unsigned long long clk_c0 = 0, clk_r0 = 0;
    if (stamps) {
      clk_c0 = __builtin_amdgcn_s_memtime();
      clk_r0 = __builtin_amdgcn_s_memrealtime();
    }
    const int wm0 = (wave / Cfg::WGN) * Cfg::WTM;
    const int wn0 = (wave % Cfg::WGN) * Cfg::WTN;

    // ---- DMA staging: per-lane chunk assignment (independent of k) ----
    const int a_row0 = wave * Cfg::A_INSTR * Cfg::A_ROWS_PER_INSTR + lane / Cfg::A_ROW_CHUNKS;
    const int a_phys = lane % Cfg::A_ROW_CHUNKS;
    const int b_row0 = wave * Cfg::B_INSTR * Cfg::B_ROWS_PER_INSTR + lane / Cfg::B_ROW_CHUNKS;
    const int b_phys = lane % Cfg::B_ROW_CHUNKS;

    // DMA of K step k0 into stage `st`, one 1 KB instruction at a time (instruction d < A_INSTR: A,
    // else B). Steps past the slice are all out of range (zeros, no traffic): they keep the number
    // of DMA operations per step constant, which the vmcnt waits rely on.
    auto rsrc_a = [&](int k0) {
      if constexpr (PACKED_A) {
        static_assert(Cfg::BM == 256 && Cfg::BK == 32 && !SPLITK, "packed A is the stage image of 256 rows x 32 K");
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>(A) + static_cast<size_t>(tm) * ceil_div(K, BK) * (Cfg::A_BYTES / 2), 0, 0x7fffffff,
            kRawBufferDword3);
      } else {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(A) + static_cast<size_t>(m0) * K + k0, 0,
                                                 0x7fffffff, kRawBufferDword3);
      }
    };
    auto rsrc_b = [&](int k0) {
      if constexpr (PACKED_B) {
        // The packed weight holds B^T in 256-row blocks (g16_pack_weight). A 256-column tile streams
        // whole 16 KB blocks; a 128-column tile streams one half of each: rows 0-127 of a block are
        // its first 8 KB (chunks q < 8), rows 128-255 the second, each already the 128-row stage
        // image (the row swizzle repeats every 8 rows). Step k0 adds k0/BK blocks (16 KB) either way.
        static_assert(PACKED_A && (Cfg::BN == 256 || Cfg::BN == 128), "packed weight: the 256-row tiles");
        constexpr int kHalves = 256 / Cfg::BN;
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16*>(B) + static_cast<size_t>(tn / kHalves) * ceil_div(K, BK) * 8192 + (tn % kHalves) * 4096, 0,
            0x7fffffff, kRawBufferDword3);
      } else {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(B) + static_cast<size_t>(k0) * N + n0, 0,
                                                 0x7fffffff, kRawBufferDword3);
      }
    };
    auto dma_op = [&](int st, int k0, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, int d) {
      if (d < Cfg::A_INSTR && PACKED_A) {
        // Tile-packed A (g16_rowscale_pack_*): the stage image of step k0 is one contiguous 16 KB
        // block; instruction q of the stage copies its q-th KB. ra is based at this tile row.
        const int q = wave * Cfg::A_INSTR + d;
        // uniform part of the offset (kOob for a step past the slice) plus this lane's 16 bytes;
        // the sum of kOob and a lane part (< 16 KB) is still past the descriptor's range: zeros
        const uint32_t step_off = k0 < kend ? static_cast<uint32_t>(k0) / BK * 16384u : kOob;
        dma16(ra, sA_lds + st * Cfg::A_BYTES + q * 1024, step_off + (q * 64 + lane) * 16);
      } else if (d < Cfg::A_INSTR) {
        const int row = a_row0 + d * Cfg::A_ROWS_PER_INSTR;
        const int c = a_phys ^ Cfg::swz_a(row);
        const bool ok = (m0 + row < M) && (k0 + c * 8 < kend);
        const uint32_t off = ok ? static_cast<uint32_t>((row * K + c * 8) * 2) : kOob;
        dma16(ra, sA_lds + st * Cfg::A_BYTES + (wave * Cfg::A_INSTR + d) * 1024, off);
      } else if (PACKED_B) {
        // Packed weight (g16_pack_weight): B^T's stage image, like packed A.
        const int q = wave * Cfg::B_INSTR + (d - Cfg::A_INSTR);
        const uint32_t step_off = k0 < kend ? static_cast<uint32_t>(k0) / BK * 16384u : kOob;
        dma16(rb, sB_lds + st * Cfg::B_BYTES + q * 1024, step_off + (q * 64 + lane) * 16);
      } else {
        const int i = d - Cfg::A_INSTR;
        const int row = b_row0 + i * Cfg::B_ROWS_PER_INSTR;
        const int c = b_phys ^ Cfg::swz_b(row);
        const bool ok = (k0 + row < kend) && (n0 + c * 8 < N);
        const uint32_t off = ok ? static_cast<uint32_t>((row * N + c * 8) * 2) : kOob;
        dma16(rb, sB_lds + st * Cfg::B_BYTES + (wave * Cfg::B_INSTR + i) * 1024, off);
      }
    };
    auto dma = [&](int st, int k0) {
      const __amdgpu_buffer_rsrc_t ra = rsrc_a(k0), rb = rsrc_b(k0);
#pragma unroll
      for (int d = 0; d < Cfg::DMA_PER_STEP; ++d) dma_op(st, k0, ra, rb, d);
    };
    // Inside the K loops, B's descriptor for successive steps comes from a running pointer (row-major
    // B: one 64-bit add per step instead of a 64-bit multiply); b_run is set to the first step's base
    // before each loop, and every call advances it by one step.
    const _Float16* b_run = nullptr;
    auto rsrc_b_next = [&](int k0) {
      if constexpr (PACKED_B) {
        return rsrc_b(k0);
      } else {
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(b_run), 0, 0x7fffffff, kRawBufferDword3);
        b_run += static_cast<size_t>(BK) * N;
        return r;
      }
    };

    // ---- fragment addressing (byte offsets within a stage) ----
    // MFMA operands (both shapes): lane l holds the 8-deep k-run 8*(l/MB) .. +7 of the MFMA's K step
    // for A row l%MB (B column l%MB). A and B use the same lane -> k assignment, so the product does
    // not depend on how the instruction orders k internally.
    const int frow = lane & (MB - 1);  // A fragment row (B^T row) within a block
    const int fk = lane / MB;          // which 8-run of the MK-deep K step
    // B transposed reads: the 16-lane group g covers columns +16*(g&1) and k rows +8*(g>>1) of a
    // 32x16 step (32x32x16), or k rows +8*g of a 16x32 step (16x16x32); lane q of the group
    // addresses row q/4, columns 4*(q%4).
    const int bg = lane >> 4, bq = lane & 15;
    const int b_col_in = (Cfg::MF16 ? 0 : 16 * (bg & 1)) + 4 * (bq & 3);  // column within the block
    const int b_k_in = 8 * (Cfg::MF16 ? bg : (bg >> 1)) + (bq >> 2);      // k row within the step (first read)

    auto a_off = [&](int i, int ks) {
      const int row = wm0 + MB * i + frow;
      const int chunk = ks * (MK / 8) + fk;
      return row * (BK * 2) + ((chunk ^ Cfg::swz_a(row)) * 16);
    };
    auto b_off = [&](int j, int krow) {
      const int col = wn0 + MB * j + b_col_in;
      return krow * (BN * 2) + (((col >> 3) ^ Cfg::swz_b(krow)) * 16) + (col & 7) * 2;
    };
    // Every k row one lane reads in a step (b_k_in, +4, +MK per substep) has the same swizzle (see
    // swz_b): b_off(j, b_k_in + r) = b_off(j, b_k_in) + r * BN * 2. One LDS address per block, offset
    // by the stage base, serves all of a step's transposing reads.
    uint32_t b_tr[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) b_tr[j] = sB_lds + static_cast<uint32_t>(b_off(j, b_k_in));

    using AccT = std::conditional_t<Cfg::MF16, float4v, float16v>;
    AccT acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = AccT{};

    // Fragments of one whole K step (BK/MK MFMA substeps), double-buffered across steps: the MFMAs
    // of step j run on set j&1 while the LDS reads of step j+1 fill set (j+1)&1.
    constexpr int KS = BK / MK;
    half8 af[2][KS][TM], bf[2][KS][TN];
    // Speculative A: the largest and smallest x this lane has multiplied, per fragment row i and per
    // fp16 half of a dword (lane l's A fragments i are all of row wm0 + 32 i + l % 32). The IEEE
    // maximum/minimum propagate a NaN, so a NaN counts as above the threshold, which only costs a
    // recompute. Chains of two become v_pk_maximum3_f16 / v_pk_minimum3_f16: 4 VALU instructions per
    // 8-value fragment.
    half2v xmax[TM] = {}, xmin[TM] = {};
    auto track_amax = [&](int buf) {
      if constexpr (SPEC) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            const half8 v = af[buf][ks][i];
            const half2v d0 = __builtin_shufflevector(v, v, 0, 1), d1 = __builtin_shufflevector(v, v, 2, 3);
            const half2v d2 = __builtin_shufflevector(v, v, 4, 5), d3 = __builtin_shufflevector(v, v, 6, 7);
            xmax[i] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(xmax[i], d0), d1);
            xmax[i] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(xmax[i], d2), d3);
            xmin[i] = __builtin_elementwise_minimum(__builtin_elementwise_minimum(xmin[i], d0), d1);
            xmin[i] = __builtin_elementwise_minimum(__builtin_elementwise_minimum(xmin[i], d2), d3);
          }
      }
    };
    // The recomputation's cast: fp16_rne(x * 2^-e) of each fragment row, as one fp16 multiply by the
    // row's factor 2^-e (0 for a row whose scale is +inf): the product is exact before rounding, and
    // fp16 denormals are kept, so it is the rowscale cast's value bit for bit (e <= 24 here).
    half2v fac[TM];
    auto scale_frags = [&](int buf) {
      if constexpr (SPEC) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int i = 0; i < TM; ++i)
            af[buf][ks][i] *= __builtin_shufflevector(fac[i], fac[i], 0, 1, 0, 1, 0, 1, 0, 1);
      }
    };
    // fragment read f of a step: f = ks * (TM + TN) + (i < TM ? i : TM + j)
    // st: the ring stage of B (and of A); sta: A's stage where it differs (the resident-A tile keeps
    // every K step's A image in its own stage)
    auto frag_op = [&](int buf, int st, int f, int sta = -1) {
      const int ks = f / (TM + TN), w = f % (TM + TN);
      if (w < TM) {
        af[buf][ks][w] = *reinterpret_cast<const half8*>(&sA[sta < 0 ? st : sta][a_off(w, ks)]);
      } else if constexpr (PACKED_B) {
        // B^T stored [n][k] like A: one 16-byte read gives lane l the k-run of column l%32.
        const int j = w - TM;
        const int row = wn0 + MB * j + frow;
        const int chunk = ks * (MK / 8) + fk;
        bf[buf][ks][j] = *reinterpret_cast<const half8*>(
            &sB[st][row * (BK * 2) + ((chunk ^ Cfg::swz_a(row)) * 16)]);
      } else {
        const int j = w - TM;
        const uint32_t at = b_tr[j] + st * Cfg::B_BYTES + ks * MK * (BN * 2);
        const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds4_at(at));
        const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds4_at(at + 4 * (BN * 2)));
        bf[buf][ks][j] = __builtin_bit_cast(half8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    auto read_frags = [&](int buf, int st, int sta = -1) {
#pragma unroll
      for (int f = 0; f < KS * (TM + TN); ++f) frag_op(buf, st, f, sta);
    };
    // MFMA m of a step: m = (ks * TM + i) * TN + jj, with j = jj on even i and TN - 1 - jj on odd i
    // (a snake over the blocks), so that consecutive MFMAs always share one operand register: the
    // A fragment within a row of blocks, the B fragment across the turn. The part is power-limited
    // on random operands and the MFMA's power grows with the operand bits that toggle between
    // instructions: measured ~1 % faster than the plain row order at 4096^3, same result bits (every
    // accumulator still receives its MFMAs in K order).
    auto mfma_op = [&](int buf, int m) {
      const int ks = m / (TM * TN), i = (m / TN) % TM, jj = m % TN, j = (i & 1) ? TN - 1 - jj : jj;
      if constexpr (Cfg::MF16)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[buf][ks][i], bf[buf][ks][j], acc[i][j], 0, 0, 0);
      else
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[buf][ks][i], bf[buf][ks][j], acc[i][j], 0, 0, 0);
    };

    // Resident A: this tile's BM rows of X, scaled and cast to fp16, written as the stage images of
    // all nk K steps (row r's logical 16-byte chunk c of step j at stage j, byte r * BK * 2 +
    // ((c ^ swz_a(r)) * 16): where the DMA would put it), zeros past K and past M; s_scale[r] gets
    // the row's scale. Wavefront w casts rows 8w .. 8w+7, all of their loads in flight at once.
    auto cast_resident = [&](auto* xp) {
      if constexpr (RESIDENT) {
        using TX = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
        constexpr int EPC = 16 / static_cast<int>(sizeof(TX));                  // elements per input chunk
        constexpr int CM = (kResidentSteps * BK / EPC + kWave - 1) / kWave;      // input chunks per lane and row
        constexpr int RPW = BM / Cfg::WAVES;                                     // rows per wavefront
        constexpr int RB = RPW;                                                  // rows in flight
        const int nch = K / EPC;
        for (int b = 0; b < RPW; b += RB) {
          u32x4 v[RB][CM];
          float am[RB];
#pragma unroll
          for (int i = 0; i < RB; ++i) {
            const int grow = m0 + wave * RPW + b + i;
            const u32x4* xr = reinterpret_cast<const u32x4*>(xp + static_cast<size_t>(min(grow, M - 1)) * K);
            am[i] = 0.f;
#pragma unroll
            for (int c = 0; c < CM; ++c) {
              const int idx = lane + c * kWave;
              v[i][c] = (grow < M && idx < nch) ? xr[idx] : u32x4{0u, 0u, 0u, 0u};
            }
          }
#pragma unroll
          for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int c = 0; c < CM; ++c) am[i] = chunk_absmax(am[i], v[i][c], TX{});
#pragma unroll
          for (int i = 0; i < RB; ++i) am[i] = wave_max(am[i]);
#pragma unroll
          for (int i = 0; i < RB; ++i) {
            const int r = wave * RPW + b + i;
            int e;
            float sc;
            row_exponent(am[i], texp, e, sc);
            if (lane == 0) s_scale[r] = sc;
            unsigned char* row_base = &sA[0][0] + r * (BK * 2);
            const int sw = Cfg::swz_a(r);
#pragma unroll
            for (int c = 0; c < CM; ++c) {
              const int idx = lane + c * kWave;
              if (idx < nch) {
                if constexpr (EPC == 8) {
                  // elements 8 idx .. 8 idx + 7: step idx / 8, logical chunk idx % 8
                  *reinterpret_cast<u32x4*>(row_base + (idx >> 3) * Cfg::A_BYTES + (((idx & 7) ^ sw) << 4)) =
                      cast_scaled(v[i][c], e, TX{});
                } else {
                  // elements 4 idx .. 4 idx + 3: half idx % 2 of output chunk idx / 2
                  const int oc = idx >> 1;
                  *reinterpret_cast<u32x2*>(row_base + (oc >> 3) * Cfg::A_BYTES + (((oc & 7) ^ sw) << 4) + ((idx & 1) << 3)) =
                      cast_scaled(v[i][c], e, TX{});
                }
              }
            }
          }
        }
        // zeros for the columns past K in the last step (K % BK != 0)
        const int oc0 = K / 8, oc1 = nk * (BK / 8);
        for (int i = 0; i < RPW; ++i) {
          const int r = wave * RPW + i;
          unsigned char* row_base = &sA[0][0] + r * (BK * 2);
          for (int oc = oc0 + lane; oc < oc1; oc += kWave)
            *reinterpret_cast<u32x4*>(row_base + (oc >> 3) * Cfg::A_BYTES + (((oc & 7) ^ Cfg::swz_a(r)) << 4)) =
                u32x4{0u, 0u, 0u, 0u};
        }
      }
    };

    static_assert(NSTAGE >= 3, "three stages at least");
    constexpr int NMFMA = KS * TM * TN, NFRAG = KS * (TM + TN), NDMA = Cfg::DMA_PER_STEP;
    // ---- 4-wavefront tiles: a ring of NSTAGE stages ----
    // During step j: MFMAs of step j (its fragments are already in registers, read during step j-1),
    // LDS reads of step j+1, and DMA of step j+NSTAGE into stage j%NSTAGE -- the stage step j came
    // from, which nobody reads any more. Before the barrier that ends step j, step j+2 must have
    // landed (it is read during j+1): NSTAGE-2 younger steps of DMA may still be in flight, giving
    // each DMA NSTAGE-1 steps to arrive. The three streams are cut into PARTS slices issued
    // round-robin (DMA, MFMAs, LDS reads), so no wavefront front-loads its DMA and the memory pipes
    // see a steady trickle between barriers.
    constexpr int LAG = NSTAGE - 2;
    // One pass of the K loop over [kbeg, kend) into acc, with A streamed through the ring (RES
    // false) or cast into the resident stages first (RES true); RESCALE: the speculative path's
    // recomputation, which scales the streamed A fragments by their rows' factors before use.
    auto kloop4 = [&](auto resc, auto rescale) {
      constexpr bool RES = decltype(resc)::value;
      constexpr bool RESCALE = decltype(rescale)::value;
      // DMA instructions per step: A and B, or B alone with resident A
      constexpr int DMA0 = RES ? Cfg::A_INSTR : 0;
      constexpr int PARTS = NDMA - DMA0;
      if constexpr (RES) {
        if (nk > 0) {
#pragma unroll
          for (int s = 0; s < NSTAGE; ++s) {
            const int k0 = kbeg + s * BK;
            const __amdgpu_buffer_rsrc_t ra = rsrc_a(k0), rb = rsrc_b(k0);
#pragma unroll
            for (int d = DMA0; d < NDMA; ++d) dma_op(s, k0, ra, rb, d);
          }
        }
        // While B's first stages land: the cast of this tile's rows into the resident A stages.
        if (x_f32) cast_resident(static_cast<const float*>(X));
        else cast_resident(static_cast<const _Float16*>(X));
      } else {
        if (nk > 0) {
#pragma unroll
          for (int s = 0; s < NSTAGE; ++s) dma(s, kbeg + s * BK);
        }
      }
      wait_dma_le<LAG * PARTS>();  // steps 0 and 1 have landed
      __syncthreads();
      if (nk > 0) read_frags(0, 0);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();  // every wavefront holds step 0 in registers: stage 0 may be refilled
      // Step j on fragment buffer H (a compile-time constant, so two steps make one loop trip). The
      // loop body has no branches: a conditional step or a conditional read inside it made the
      // compiler copy accumulators between AGPRs and VGPRs on every trip (measured: ~3x slower
      // steps). The last step's reads of step j+1 are harmless: they read a stage inside the ring
      // (zeros or stale data) into the buffer no MFMA uses afterwards.
      auto step = [&](auto hc, int j) {
        constexpr int H = decltype(hc)::value;
        const int kd = kbeg + (j + NSTAGE) * BK;
        const int std_ = j % NSTAGE, stf = (j + 1) % NSTAGE;
        // resident A: step j+1's own stage (the last step reads an in-range stage it does not use)
        const int sta = RES ? (j + 1 < nk ? j + 1 : j) : -1;
        const __amdgpu_buffer_rsrc_t ra = rsrc_a(kd), rb = rsrc_b_next(kd);
        if constexpr (RESCALE) scale_frags(H);
#pragma unroll
        for (int p = 0; p < PARTS; ++p) {
          dma_op(std_, kd, ra, rb, DMA0 + p);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int m = p * NMFMA / PARTS; m < (p + 1) * NMFMA / PARTS; ++m) mfma_op(H, m);
#pragma unroll
          for (int f = p * NFRAG / PARTS; f < (p + 1) * NFRAG / PARTS; ++f) frag_op(H ^ 1, stf, f, sta);
          __builtin_amdgcn_sched_barrier(0);
        }
        // step j's A fragments (streamed x), after the step's MFMAs have been issued on them
        if constexpr (SPEC && !RES && !RESCALE) track_amax(H);
        wait_dma_le<LAG * PARTS>();  // step j+2 has landed (this wavefront's part)
        __syncthreads();            // ... every wavefront's part; step j+1 is in registers
      };
      b_run = B + static_cast<size_t>(kbeg + NSTAGE * BK) * N + n0;
      int it = 0;
      for (; it + 1 < nk; it += 2) {
        step(std::integral_constant<int, 0>{}, it);
        step(std::integral_constant<int, 1>{}, it + 1);
      }
      if (it < nk) step(std::integral_constant<int, 0>{}, it);
    };
    if constexpr (Cfg::WAVES == 8) {
      // Ping-pong schedule for two wavefronts per SIMD. Wavefronts 0-3 (group 0) and 4-7 (group 1)
      // land one of each on every SIMD. Each wavefront alternates a memory phase M_j (fragment reads
      // of step j from LDS, DMA of step j+D into the ring) and a compute phase C_j (the MFMAs of
      // step j), with a workgroup barrier after every phase; group 1 starts one phase late, so on
      // every SIMD one wavefront streams MFMAs while the other one waits on memory.
      //   Ring hazards, with D = NSTAGE - 2 (the DMA runs two steps ahead): the DMA issued in M_j
      // writes stage (j+D)%NSTAGE, which last held step j-2. Group 0 read step j-2 in M_{j-2} and
      // group 1 one phase later; a wavefront's reads of a step have returned before the first MFMA
      // of that step's compute phase, which waits for them (the compiler places that wait), and
      // group 1's C_{j-2} ends with a barrier that precedes the opening of M_j for either group.
      // So the memory phase does not wait for its own LDS reads before its closing barrier: they
      // land while the barrier waits for the other group's MFMAs (measured at 4096^3: loop 148.9k ->
      // 137.7k shader cycles, 126.6 -> 123.7 us per cast + GEMM step, bitwise the same output;
      // with the DMA three steps ahead the next DMA would overwrite the stage group 1 has just
      // read, so that form needs the wait). The fragment reads of M_j need every wavefront's DMA
      // of step j: each wavefront waits for its own at the end of M_{j-1}, and the barrier after
      // that phase publishes it to the group that reads next.
      constexpr int D = NSTAGE - 2;
      const int grp = wave >> 2;
      if (nk > 0) {
#pragma unroll
        for (int s = 0; s < D; ++s) dma(s, kbeg + s * BK);
      }
      wait_dma_le<(D - 1) * NDMA>();  // step 0 has landed
      b_run = B + static_cast<size_t>(kbeg + D * BK) * N + n0;
      phase_barrier();
      if (grp == 1) phase_barrier();
      for (int j = 0; j < nk; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        {
          // The memory phase interleaves its fragment reads (LDS) and its DMA issue (texture path):
          // NFRAG / NDMA reads, then one DMA instruction, NDMA times, then any reads left over. On
          // the 256x256 tile at 4096^3 (12 reads, 4 DMA) this ran 0.4-0.6 % faster than all reads
          // before all DMA, with the same result bits; every form that issues a DMA before the
          // first reads ran 1.5-3 % slower.
          const int kd = kbeg + (j + D) * BK;
          const __amdgpu_buffer_rsrc_t ra = rsrc_a(kd), rb = rsrc_b_next(kd);
          constexpr int PER = NFRAG / NDMA;
#pragma unroll
          for (int d = 0; d < NDMA; ++d) {
#pragma unroll
            for (int f = d * PER; f < (d + 1) * PER; ++f) frag_op(0, j % NSTAGE, f);
            dma_op((j + D) % NSTAGE, kd, ra, rb, d);
          }
#pragma unroll
          for (int f = NDMA * PER; f < NFRAG; ++f) frag_op(0, j % NSTAGE, f);
        }
        wait_dma_le<(D - 1) * NDMA>();  // step j+1 has landed (this wavefront's part)
        phase_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < NMFMA; ++m) mfma_op(0, m);
        __builtin_amdgcn_sched_barrier(0);
        phase_barrier();
      }
      if (grp == 0) phase_barrier();  // every wavefront passes the same number of barriers
    } else {
      if constexpr (RESIDENT) kloop4(std::true_type{}, std::false_type{});
      else kloop4(std::false_type{}, std::false_type{});
    }
    wait_dma_le<0>();  // no DMA may still be writing LDS past this point
    if (stamps && tid == 0) {
      g_loop_clock[0] = __builtin_amdgcn_s_memtime() - clk_c0;
      g_loop_clock[1] = __builtin_amdgcn_s_memrealtime() - clk_r0;
    }

    // ---- speculative A: recompute the tile where some |x| exceeded the threshold ----
    bool respec = false;  // acc comes from the rescaled A, with the row scales in s_scale
    auto zero_acc = [&]() {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = AccT{};
    };
    // max with a NaN in either operand giving NaN
    auto nan_max = [](float a, float b) { return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b); };
    // this lane's rows' |max| over the K range it has multiplied (lanes l and l ^ 32 hold the same
    // row, different k), NaN where a NaN was seen
    float ramax[TM];
    int over = 0;  // some row of this slice exceeded the threshold or held a NaN (the workgroup agrees)
    if constexpr (SPEC) {
      // the largest fp16 value not above the threshold; a NaN fails the comparison
      const float t = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(tbits)));
      bool within = true;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        float a = nan_max(nan_max(static_cast<float>(xmax[i].x), static_cast<float>(xmax[i].y)),
                          nan_max(-static_cast<float>(xmin[i].x), -static_cast<float>(xmin[i].y)));
        a = nan_max(a, __shfl_xor(a, 32));
        ramax[i] = a;
        within = within && a <= t;
      }
      over = __syncthreads_or(within ? 0 : 1);
    }
    // With s_rowmax holding every row's |max| (NaN where a NaN was seen): the rows' exponents, exactly
    // as the rowscale cast derives them, into s_scale (2^e) and this lane's factors fac (2^-e). A
    // row with a NaN gets its |max| over all of K from x itself, NaN dropped as the cast drops it.
    auto row_factors = [&]() {
      if constexpr (SPEC) {
        for (int r = wave; r < BM; r += Cfg::WAVES) {
          const float v = s_rowmax[r];
          if (v != v) {
            float am = 0.f;
            if (m0 + r < M) {
              const u32x4* xr = reinterpret_cast<const u32x4*>(A + static_cast<size_t>(m0 + r) * K);
              for (int idx = lane; idx < K / 8; idx += kWave) am = chunk_absmax(am, xr[idx], _Float16{});
            }
            am = wave_max(am);
            if (lane == 0) s_rowmax[r] = am;
          }
        }
        __syncthreads();
        if (tid < BM) {
          int e;
          float sc;
          row_exponent(s_rowmax[tid], texp, e, sc);
          s_scale[tid] = sc;
          s_rowmax[tid] = e == kInfExp ? 0.f : ldexpf(1.f, -e);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const _Float16 f = static_cast<_Float16>(s_rowmax[wm0 + 32 * i + (lane & 31)]);
          fac[i] = half2v{f, f};
        }
      }
    };
    // the wavefronts of the first column hold every row once: lanes < 32 write them
    const bool row_writer = wave % Cfg::WGN == 0 && lane < 32;
    // a recomputation is remembered for the weight (the host routes its next calls around it)
    auto note_miss = [&]() {
      if (spec_miss != nullptr && tid == 0) __hip_atomic_store(spec_miss, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    };
    if constexpr (SPEC && !SPLITK) {
      if (over) {
        respec = true;
        note_miss();
        if (row_writer) {
#pragma unroll
          for (int i = 0; i < TM; ++i) s_rowmax[wm0 + 32 * i + lane] = ramax[i];
        }
        __syncthreads();
        row_factors();
        zero_acc();
        kloop4(std::false_type{}, std::true_type{});
        wait_dma_le<0>();
      }
    }

    // ---- split-K: publish this slice, let the last slice reduce ----
    if constexpr (SPLITK) {
      constexpr uint32_t TILE_BYTES = BM * BN * 4;
      // Each wavefront stores its accumulators in its own register order: slot s of the wavefront is
      // float4 piece q of accumulator (i, j), s = (i * TN + j) * QV + q.
      constexpr int QV = sizeof(AccT) / sizeof(float4v);  // 4 for 32x32 blocks, 1 for 16x16 blocks
      constexpr int SLOTS = TM * TN * QV;
      auto piece = [&](int s) -> float4v {
        const int b = s / QV, q = s % QV;
        if constexpr (QV == 1) {
          return acc[b / TN][b % TN];
        } else {
          const AccT& a = acc[b / TN][b % TN];
          return float4v{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
        }
      };
      auto set_piece = [&](int s, float4v v) {
        const int b = s / QV, q = s % QV;
        if constexpr (QV == 1) {
          acc[b / TN][b % TN] = v;
        } else {
          AccT& a = acc[b / TN][b % TN];
          a[4 * q] = v.x;
          a[4 * q + 1] = v.y;
          a[4 * q + 2] = v.z;
          a[4 * q + 3] = v.w;
        }
      };
      const __amdgpu_buffer_rsrc_t slices =
          coherent_rsrc(part + static_cast<size_t>(tile) * ksplit * (BM * BN), static_cast<uint32_t>(ksplit) * TILE_BYTES);
      auto slot_off = [&](int z, int s) {
        return static_cast<uint32_t>(z) * TILE_BYTES + static_cast<uint32_t>((wave * SLOTS + s) * 64 + lane) * 16u;
      };
      // the speculative path's rows' |max| of slice z: the first BM floats of its partial tile
      auto rowmax_slot = [&](int zz) { return part + (static_cast<size_t>(tile) * ksplit + zz) * (BM * BN); };
      if (SPEC && over) {
        // the last slice recomputes this tile: publish the rows' |max| in place of the partial tile
        if (row_writer) {
#pragma unroll
          for (int i = 0; i < TM; ++i) store_coherent(rowmax_slot(z) + wm0 + 32 * i + lane, ramax[i]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) store_coherent4(slices, slot_off(z, s), piece(s));
      }
      if constexpr (SPEC) {
        const uint32_t total = arrive_add_coherent(counters + tile * kCounterStride,
                                                   1u + (over ? (1u << (kSpecShift + z)) : 0u));
        if ((total & ((1u << kSpecShift) - 1u)) != static_cast<uint32_t>(ksplit)) return;
        respec = (total >> kSpecShift) != 0u;
        if (respec) {
          // a row's |max| over K: the largest over the slices that saw a value above the threshold
          // (the others hold none, so they cannot raise a row's exponent above 0)
          const uint32_t mask = total >> kSpecShift;
          if (tid < BM) {
            float m = 0.f;
            for (int zz = 0; zz < ksplit; ++zz)
              if ((mask >> zz) & 1u) m = nan_max(m, load_coherent(rowmax_slot(zz) + tid));
            s_rowmax[tid] = m;
          }
          __syncthreads();
        }
      } else {
        if (!arrive_last_coherent(counters + tile * kCounterStride, static_cast<uint32_t>(ksplit))) return;
      }
      // Slices are added in slice order (every slice, this one's included, is read back from the
      // workspace), so each output is the same sum whichever slice arrives last.
      if (SPEC && respec) {
        // Some slice's A exceeded the threshold: recompute every slice with the rescaled A and add
        // them in slice order, exactly as the reduction below adds the published slices.
        if constexpr (SPEC) {
          static_assert(SLOTS <= 16, "the 4-wavefront tiles");
          note_miss();
          row_factors();
          float4v sum[SLOTS];
#pragma unroll
          for (int s = 0; s < SLOTS; ++s) sum[s] = float4v{0.f, 0.f, 0.f, 0.f};
          for (int zz = 0; zz < ksplit; ++zz) {
            kbeg = zz * kchunk;
            kend = min(K, kbeg + kchunk);
            nk = kend > kbeg ? ceil_div(kend - kbeg, BK) : 0;
            zero_acc();
            kloop4(std::false_type{}, std::true_type{});
            wait_dma_le<0>();
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) sum[s] += piece(s);
          }
#pragma unroll
          for (int s = 0; s < SLOTS; ++s) set_piece(s, sum[s]);
        }
      } else if constexpr (SLOTS <= 16) {
        // ZB slices' loads in flight at a time
        constexpr int ZB = (128 / (SLOTS * 4)) < 1 ? 1 : ((128 / (SLOTS * 4)) > 8 ? 8 : (128 / (SLOTS * 4)));
        float4v sum[SLOTS];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) sum[s] = float4v{0.f, 0.f, 0.f, 0.f};
        for (int z0 = 0; z0 < ksplit; z0 += ZB) {
          float4v v[ZB][SLOTS];
#pragma unroll
          for (int b = 0; b < ZB; ++b)
#pragma unroll
            for (int s = 0; s < SLOTS; ++s)
              v[b][s] = z0 + b < ksplit ? load_coherent4(slices, slot_off(z0 + b, s)) : float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int b = 0; b < ZB; ++b)
#pragma unroll
            for (int s = 0; s < SLOTS; ++s)
              if (z0 + b < ksplit) sum[s] += v[b][s];
        }
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) set_piece(s, sum[s]);
      } else {
        // The 256x256 tile: its accumulators fill most of the register file, so the sums build up in
        // the accumulators themselves, kCh slots at a time, two slices' loads in flight.
        constexpr int kCh = 8;
        static_assert(SLOTS % kCh == 0, "whole chunks");
#pragma unroll
        for (int c0 = 0; c0 < SLOTS; c0 += kCh) {
          float4v s[kCh];
#pragma unroll
          for (int q = 0; q < kCh; ++q) s[q] = float4v{0.f, 0.f, 0.f, 0.f};
          for (int z0 = 0; z0 < ksplit; z0 += 2) {
            float4v v0[kCh], v1[kCh];
#pragma unroll
            for (int q = 0; q < kCh; ++q) {
              v0[q] = load_coherent4(slices, slot_off(z0, c0 + q));
              v1[q] = z0 + 1 < ksplit ? load_coherent4(slices, slot_off(z0 + 1, c0 + q)) : float4v{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int q = 0; q < kCh; ++q) {
              s[q] += v0[q];
              if (z0 + 1 < ksplit) s[q] += v1[q];
            }
          }
#pragma unroll
          for (int q = 0; q < kCh; ++q) set_piece(c0 + q, s[q]);
        }
      }
      reset_counter(counters + tile * kCounterStride);
    }

    // ---- epilogue: C = rscale[row] * acc + bias[col] ----
    // Each wavefront moves its accumulators, one 32x32 region at a time, through a private 4 KB LDS
    // scratch so that every lane ends up with 4 consecutive columns of one row: the result leaves in
    // 16-byte (fp32) or 8-byte (fp16) stores, 4x fewer store instructions than one value per lane.
    //   32x32x16 layout (a region is one block): lane l, register r -> column l%32, row
    //   8*(r/4) + 4*(l/32) + r%4. Rows R and R+4 meet in one write; storing row R at physical row
    //   R ^ ((R >> 2) & 1) gives them different bank halves.
    //   16x16x32 layout (a region is 2x2 blocks a, b): lane l, register r -> column 16b + l%16, row
    //   16a + 4*(l/16) + r. One write covers rows 4g + r of the four 16-lane groups g; the same row
    //   swizzle plus column ^ 16*((R >> 3) & 1) puts the four groups on four distinct 16-bank ranges.
    // The read-back (two rows of 8 lanes per 16 lanes) hits both bank halves whole in either layout.
    //   The rows and columns a lane stores are the same in every region (row lane / 8 + 8 q, columns
    // 4 (lane % 8) .. +3), so its row scales and column biases are loaded once, before the first
    // store. Loaded next to each store, every store waited for them, and so (vmcnt counts stores as
    // well) for the store before it: 32 memory round trips in a row per wavefront, ~5.5 us of each
    // 256x256 tile's epilogue even with the stores taken out.
    constexpr int ERI = Cfg::WTM / 32, ERJ = Cfg::WTN / 32;
    float erow[ERI][4];
    float4v ecol[ERJ];
#pragma unroll
    for (int ri = 0; ri < ERI; ++ri)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int grow = m0 + wm0 + 32 * ri + (lane >> 3) + 8 * q;
        erow[ri][q] = (RESIDENT || respec) ? s_scale[grow - m0]
                                           : (SPEC ? 1.f : (rscale != nullptr && grow < M ? rscale[grow] : 1.f));
      }
#pragma unroll
    for (int rj = 0; rj < ERJ; ++rj) {
      const int gcol = n0 + wn0 + 32 * rj + (lane & 7) * 4;
      ecol[rj] = bias != nullptr && gcol < N ? float4v{bias[gcol], bias[gcol + 1], bias[gcol + 2], bias[gcol + 3]}
                                             : float4v{0.f, 0.f, 0.f, 0.f};
    }
    // Those loads have returned before the first (bounds-guarded) store. Otherwise the compiler,
    // which cannot tell how many of the guarded stores were issued, waits for all of them (vmcnt
    // 0) before every store that uses a loaded value: the same chain of round trips again.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    // A persistent grid (more tiles than workgroups) stores C non-temporally: its stores overlap
    // other workgroups' main loops, and those store streams drain faster past the L2 (65536 x 768 x
    // 3072: 329 -> 308 us; 65536 x 768 x 768: 90.9 -> 87.5). A one-round grid keeps plain stores
    // (4096^3: 103.2 -> 105.3 us non-temporal, every workgroup storing at once).
    const bool stream_c = ntiles > static_cast<int>(gridDim.x);
    __syncthreads();  // every wavefront's DMA has drained: the stages are free for scratch
    float* scr = reinterpret_cast<float*>(&sB[0][0] + wave * 4096);
    static_assert(Cfg::B_BYTES * NSTAGE >= 4096 * Cfg::WAVES, "scratch fits in the B stages");
    auto phys = [](int row, int col) {
      return (row ^ ((row >> 2) & 1)) * 32 + (Cfg::MF16 ? (col ^ (16 * ((row >> 3) & 1))) : col);
    };
#pragma unroll
    for (int ri = 0; ri < ERI; ++ri) {
      // The non-temporal stores go through a buffer descriptor based at the region's first row
      // (offsets < 32 N elements: below 2^31 bytes for N <= G16_GEMM_MAX_N); as a buffer store with
      // its cache policy an immediate, the compiler cannot merge it with the plain store (a
      // nontemporal global store in one branch and a plain one in the other became one plain store).
      const __amdgpu_buffer_rsrc_t crsrc = __builtin_amdgcn_make_buffer_rsrc(
          static_cast<char*>(Cv) + static_cast<size_t>(m0 + wm0 + 32 * ri) * N * (OUT_F16 ? 2 : 4), 0, 0x7fffffff,
          kRawBufferDword3);
#pragma unroll
      for (int rj = 0; rj < ERJ; ++rj) {
        if constexpr (Cfg::MF16) {
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
              for (int r = 0; r < 4; ++r) scr[phys(16 * a + 4 * fk + r, 16 * b + frow)] = acc[2 * ri + a][2 * rj + b][r];
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) scr[phys(8 * (r >> 2) + 4 * fk + (r & 3), frow)] = acc[ri][rj][r];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int id = lane + 64 * q;
          const int row = id >> 3, c4 = (id & 7) * 4;
          float4v v = *reinterpret_cast<const float4v*>(&scr[phys(row, c4)]);
          const int grow = m0 + wm0 + 32 * ri + row;
          const int gcol = n0 + wn0 + 32 * rj + c4;
          if (grow < M && gcol < N) {  // N % 8 == 0: a 4-column chunk is all in or all out
            v = v * erow[ri][q] + ecol[rj];
            const uint32_t coff = static_cast<uint32_t>(row) * static_cast<uint32_t>(N) + static_cast<uint32_t>(gcol);
            if constexpr (OUT_F16) {
              const half4 h = {static_cast<_Float16>(v.x), static_cast<_Float16>(v.y), static_cast<_Float16>(v.z),
                               static_cast<_Float16>(v.w)};
              if (stream_c)
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, h), crsrc, static_cast<int>(coff * 2u), 0, kCpolNt);
              else
                *reinterpret_cast<half4*>(static_cast<_Float16*>(Cv) + static_cast<size_t>(grow) * N + gcol) = h;
            } else {
              if (stream_c)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), crsrc, static_cast<int>(coff * 4u), 0, kCpolNt);
              else
                *reinterpret_cast<float4v*>(static_cast<float*>(Cv) + static_cast<size_t>(grow) * N + gcol) = v;
            }
          }
        }
      }
    }
    // The stages (and the epilogue scratch in them) are free before the next tile's DMA: every
    // wavefront's scratch reads have returned. Its stores need not have: they drain while the next
    // tile's first DMA is in flight (__syncthreads() would wait for them here).
    if (work + static_cast<int>(gridDim.x) < ntiles) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      phase_barrier();
    }
  }
}

__global__ void copy_loop_clock(unsigned long long* dst) {
  dst[0] = g_loop_clock[0];
  dst[1] = g_loop_clock[1];
}

enum class Tile { T256, T256N, T128, T64, T32, T64x64 };

struct Plan {
  Tile tile;
  int bm, bn;
  int ntm, ntn;
  int ks = 0;  // the split the tile was chosen with (the modelled choice below); 0: the planner's rule
};

// The 4-wavefront tiles (32x32x16 MFMA blocks, one barrier per K step): the ones the speculative
// fp16 route runs on.
inline bool four_wave(Tile t) { return t == Tile::T128 || t == Tile::T64 || t == Tile::T32 || t == Tile::T64x64; }

struct KSplit {
  int ksplit;
  int kchunk;
};

KSplit ksplit_for(int K, int ksplit) {
  if (K <= 0 || ksplit <= 1) return {1, K > 0 ? K : 0};
  const int kchunk = ceil_div(ceil_div(K, ksplit), kSplitAlign) * kSplitAlign;
  return {ceil_div(K, kchunk), kchunk};
}

// Compute units of device `dev` (cached per device; 256, the MI355X count, if the query fails).
int cus_of_device(int dev) {
  static int cache[64] = {};
  if (dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    cache[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cache[dev];
}

// Compute units of the device that owns `stream` (the null stream: the current device), for the
// entry points that take no CU count of their own.
int stream_cus(hipStream_t stream) {
  int dev = 0;
  if (stream == nullptr || hipStreamGetDevice(stream, &dev) != hipSuccess) {
    if (hipGetDevice(&dev) != hipSuccess) return 256;
  }
  return cus_of_device(dev);
}

// Compute units of the current device, for the size queries when the caller passes num_cus <= 0.
int current_cus() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess ? cus_of_device(dev) : 256;
}

// Size limits of the 32-bit buffer offsets the DMA uses. A row-major A offset is at most
// BM * K * 2 bytes past its tile row (BM <= 256), a packed A or B offset at most 16 KB per K step of
// 32 past its tile row, and a row-major B offset at most BK * N * 2 bytes (BK <= 64) past its K
// step; every one must stay below the descriptors' 2^31 - 1 byte range (an offset past it reads
// zeros, which would make an oversized operand's product silently wrong).
constexpr int kMaxK = G16_GEMM_MAX_K;
constexpr int kMaxN = G16_GEMM_MAX_N;

// Tile and split of the 4-wavefront tiles (32x128, 64x128, 64x64, 128x128) for M > 64 outside the
// 256-row tiles' range: the pair with the least modelled time among those whose grid fits one round
// on the CUs (1 to 8 slices of >= 256 K). Per tile, time (us) = a + b * KB + c * T + [split] * (d
// + e * P + f * g / CUs + h * [tiles % 8 != 0] * T), where KB = the A and B bytes one workgroup
// streams, (BM + BN) * kchunk * 2 / 1024; g = workgroups (tiles x slices); T = g * KB / 1024, the
// grid's traffic; P = the KB of fp32 partial tiles the last slice reads back; and the h term is the
// traffic of a split grid without the XCD-grouped tile order (which split grids get only when the
// tile count is a multiple of 8). Least-squares fit of graph-timed kernels on 256 CUs: 148
// shapes, M = 72..1024, K = 264..14336, N = 264..14336, every tile and split that fits one round
// (133 of them have such a grid). Fitted on one half of the shapes, its picks on the other half took
// 0.56 % more time than the best measured pairs (40 random halvings; at most 0.77 %); without the
// 64x64 tile the best pairs themselves take 2.6 % more, and a model of the other three tiles 3.6 %.
// Earlier rules took 7.8 % more (the 32- and 64-row tiles only for K <= 3072) and up to 2x on some
// shapes, e.g. 192 x 4096 x 512: 18.0 us on 128x128 tiles split 4 ways against 9.4 on 32x128 split
// 8 ways; the 64x64 tile: 160 x 1536 x 11008 (M x K x N) 17.9 -> 12.9 us against 64x128 tiles
// split 7 ways; 1024^3 unsplit 9.4 -> 8.2 (modelled) against 32x128.
struct TileCost {
  Tile tile;
  int bm, bn;
  double a, b, c, d, e, f, h;
};
constexpr TileCost kTileCost[4] = {
    {Tile::T32, 32, 128, 4.8257, 0.011467, 0.012217, 0.35769, 0.01376, 1.218, 0.046066},
    {Tile::T64, 64, 128, 6.1411, 0.011029, 0.016788, 0.31265, 0.012935, 2.0704, 0.042793},
    {Tile::T64x64, 64, 64, 4.4223, 0.013086, 0.0069148, 1.8756, 0.0031762, 0.98682, 0.03103},
    {Tile::T128, 128, 128, 7.2055, 0.013027, 0.01719, 0.43912, 0.013514, 2.9942, 0.016906},
};

bool modelled_tile(int M, int N, int K, int num_cus, Plan& out) {
  double best = 0.0;
  bool found = false;
  for (const TileCost& c : kTileCost) {
    const long tiles = static_cast<long>(ceil_div(M, c.bm)) * ceil_div(N, c.bn);
    for (int want = 1; want <= 8; ++want) {
      if (want > 1 && K / want < 256) break;
      const KSplit sp = ksplit_for(K, want);
      if (sp.ksplit != want) continue;  // fewer slices than asked: counted at that count
      const long g = tiles * sp.ksplit;
      if (g > num_cus) break;
      const double kb = (c.bm + c.bn) * static_cast<double>(sp.kchunk) * 2.0 / 1024.0;
      const double traffic = static_cast<double>(g) * kb / 1024.0;
      const double part = sp.ksplit * c.bm * c.bn * 4 / 1024.0;
      double t = c.a + c.b * kb + c.c * traffic;
      if (sp.ksplit > 1)
        t += c.d + c.e * part + c.f * static_cast<double>(g) / num_cus + (tiles % 8 != 0 ? c.h * traffic : 0.0);
      if (!found || t < best) {
        best = t;
        out = Plan{c.tile, c.bm, c.bn, ceil_div(M, c.bm), ceil_div(N, c.bn), sp.ksplit};
        found = true;
      }
    }
  }
  return found;
}

// The same tile with or without a split: a split only spreads K over more workgroups. M <= 64 takes
// the 32x128 or 64x128 tile (below). Large outputs take the 256x256 tile once it gives more than
// half the CUs a workgroup; just below that (3/8 to 1/2 of the CUs), the 256x128 tile on the same
// schedule fills them instead (2048 x 4096^2, 128 tiles of 256^2 on 256 CUs: 89 us, 256 tiles of
// 256x128: 76-82 us; with 144 tiles of 256^2 the 256x128 grid would overflow the CUs: 93 vs 128 us).
// Below that, the modelled 4-wavefront choice above; where no 4-wavefront grid fits one round, the
// 128x128 tile unsplit.
Plan choose_tile(int M, int N, int K, int num_cus) {
  Plan p{};
  const long t256 = static_cast<long>(ceil_div(M, 256)) * ceil_div(N, 256);
  if (M <= 32 || (M <= 64 && 4L * ceil_div(N, 128) <= num_cus) ||
      (M <= 64 && K < kMinSplitK && 2L * ceil_div(N, 128) <= num_cus)) {
    // M = 33..64 on two rows of 32x128 tiles while they fill at most half the CUs, so the split
    // still doubles them (graph-timed, M x N x K: 64 x 1024^2 8.6 -> 6.8 us, 64 x 1024 x 4096
    // 11.4 -> 9.7, 64 x 4096^2 13.9 -> 11.9, 64 x 4096 x 11008 23.6 -> 21.5); with more tiles than
    // that, 64x128 tiles split twice beat unsplit 32x128 ones (64 x 11008 x 4096: 21.4 vs 31.3 us),
    // except at K below kMinSplitK, which is not split: then 32x128 tiles wherever their grid fits
    // one round (40 x 11008 x 512: 6.6 us against 9.7 on 64x128 tiles split twice).
    p.tile = Tile::T32; p.bm = 32; p.bn = 128;
  } else if (M <= 64) {
    p.tile = Tile::T64; p.bm = 64; p.bn = 128;
  } else if (M >= 1024 && N >= 256 && 2 * t256 > num_cus) {
    p.tile = Tile::T256; p.bm = 256; p.bn = 256;
  } else if (M >= 1024 && N >= 256 && 8 * t256 > 3 * num_cus) {
    p.tile = Tile::T256N; p.bm = 256; p.bn = 128;
  } else if (modelled_tile(M, N, K, num_cus, p)) {
    return p;
  } else if (M >= 512 && N >= 256 && K >= 1024 && 5L * ceil_div(M, 256) * 256 <= 6L * M &&
             (K >= 4096 || static_cast<long>(ceil_div(M, 256)) * ceil_div(N, 128) > num_cus)) {
    // No 4-wavefront grid fits one round: the 256-row tiles on their packed route win over 128x128
    // tiles that need 1.25 rounds or more -- the 256x128 tile where its grid fits one round and K
    // is long, else the 256x256 one (mm_t, fp32 x, graph-timed, M x N x K: 1280 x 4096^2 78.9 ->
    // 72.9 us, 1280 x 4096 x 11008 210 -> 181 on 256x128; 768 x 11008 x 4096 126.7 -> 96.0, 640 x
    // 14336 x 4096 117.8 -> 97.2 on 256x256; plain kernels at short K: 768 x 11008 x 2048 61.7 ->
    // 54.6, 768 x 11008 x 3072 87.3 -> 71.2, 640 x 14336 x 2048 61.6 -> 54.6 on 256x256, while 256x128
    // tiles lose or tie there: 1280 x 4096 x 2048 39.7 vs 40.5). Not where more than a fifth of the
    // last tile row would be padding (600 x 11008 x 4096, fp16 x, 92.7 -> 97.6), nor below K =
    // 1024 (1100 x 4096 x 264: 17.5 -> 18.5 on 256x128); fp16 x at K = 4096 loses a little, since
    // its one-launch route needs a 4-wavefront tile (1280 x 4096^2: 69.8 -> 72.7).
    if (K >= 4096 && static_cast<long>(ceil_div(M, 256)) * ceil_div(N, 128) <= num_cus) {
      p.tile = Tile::T256N; p.bm = 256; p.bn = 128;
    } else {
      p.tile = Tile::T256; p.bm = 256; p.bn = 256;
    }
  } else {
    p.tile = Tile::T128; p.bm = 128; p.bn = 128;
  }
  p.ntm = ceil_div(M, p.bm);
  p.ntn = ceil_div(N, p.bn);
  return p;
}

template <bool OUT_F16>
using GemmFn = void (*)(const _Float16*, const _Float16*, void*, const float*, const float*, float*, uint32_t*, int,
                        int, int, int, int, int, int, const void*, int, int, int, uint32_t*);

template <bool OUT_F16>
GemmFn<OUT_F16> gemm_fn(Tile t, bool splitk, bool packed, bool packed_b, bool resident = false, bool spec = false) {
  if (spec) {
    // speculative fp16 A on the 4-wavefront tiles
    if (splitk) {
      switch (t) {
        case Tile::T128: return hgemm_kernel<Cfg128, OUT_F16, true, false, false, false, true>;
        case Tile::T64: return hgemm_kernel<Cfg64, OUT_F16, true, false, false, false, true>;
        case Tile::T64x64: return hgemm_kernel<Cfg64x64, OUT_F16, true, false, false, false, true>;
        default: return hgemm_kernel<Cfg32, OUT_F16, true, false, false, false, true>;
      }
    }
    switch (t) {
      case Tile::T128: return hgemm_kernel<Cfg128, OUT_F16, false, false, false, false, true>;
      case Tile::T64: return hgemm_kernel<Cfg64, OUT_F16, false, false, false, false, true>;
      case Tile::T64x64: return hgemm_kernel<Cfg64x64, OUT_F16, false, false, false, false, true>;
      default: return hgemm_kernel<Cfg32, OUT_F16, false, false, false, false, true>;
    }
  }
  if (resident) return hgemm_kernel<Cfg32, OUT_F16, false, false, false, true>;
  if (packed_b)
    return t == Tile::T256N ? hgemm_kernel<Cfg256n, OUT_F16, false, true, true> : hgemm_kernel<Cfg256, OUT_F16, false, true, true>;
  if (packed) return t == Tile::T256N ? hgemm_kernel<Cfg256n, OUT_F16, false, true> : hgemm_kernel<Cfg256, OUT_F16, false, true>;
  if (splitk) {
    switch (t) {
      case Tile::T256: return hgemm_kernel<Cfg256, OUT_F16, true>;
      case Tile::T256N: return hgemm_kernel<Cfg256n, OUT_F16, true>;
      case Tile::T128: return hgemm_kernel<Cfg128, OUT_F16, true>;
      case Tile::T64: return hgemm_kernel<Cfg64, OUT_F16, true>;
      case Tile::T64x64: return hgemm_kernel<Cfg64x64, OUT_F16, true>;
      default: return hgemm_kernel<Cfg32, OUT_F16, true>;
    }
  }
  switch (t) {
    case Tile::T256: return hgemm_kernel<Cfg256, OUT_F16, false>;
    case Tile::T256N: return hgemm_kernel<Cfg256n, OUT_F16, false>;
    case Tile::T128: return hgemm_kernel<Cfg128, OUT_F16, false>;
    case Tile::T64: return hgemm_kernel<Cfg64, OUT_F16, false>;
    case Tile::T64x64: return hgemm_kernel<Cfg64x64, OUT_F16, false>;
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

// Launches the GEMM on the tile choose_tile() picks for num_cus compute units (<= 0: the CU count of
// the stream's device), so that a caller who planned ksplit and sized the split buffers for a CU
// count gets exactly that grid.
// The activations of a resident-A launch (mm_t's GEMM path in one launch): X, its type, log2 of
// the threshold.
struct ResidentCast {
  const void* x;
  int x_f32;
  int texp;
};

// mm_t's GEMM path runs as one resident-A launch where the plan is the unsplit 32x128 tile and
// every K step of A fits in LDS.
bool resident_route(const Plan& p, int ksplit, int K) {
  return p.tile == Tile::T32 && ksplit == 1 && K > 0 && ceil_div(K, Cfg32::BK) <= kResidentSteps;
}

// A speculative launch (mm_t's GEMM path in one launch for fp16 x on the 4-wavefront tiles): log2
// of the threshold (>= kSpecMinTexp), the largest fp16 bit pattern not above it, and the weight's
// history slot (or NULL).
struct SpecA {
  int texp;
  int tbits;
  uint32_t* miss;
};
// Row exponents stay <= 16 - texp (fp16 |x| < 2^16): with texp >= -8, every factor 2^-e of the
// recomputation is an fp16 value.
constexpr int kSpecMinTexp = -8;

// Largest fp16 bit pattern whose value is <= 2^texp (0x7bff, the largest finite, above it).
int fp16_bits_at_most(int texp) {
  if (texp >= 16) return 0x7bff;
  if (texp >= -14) return (texp + 15) << 10;                // normal: exponent field texp + 15
  if (texp >= -24) return 1 << (texp + 24);                 // subnormal: 2^texp = m * 2^-24
  return 0;
}

int gemm_launch(const uint16_t* A, const uint16_t* B, void* C, bool out_f16, const float* bias, const float* rscale,
                int M, int N, int K, int ksplit, int num_cus, void* ws, size_t ws_bytes, uint32_t* counters_in,
                size_t counter_bytes_in, void* stream, bool packed = false, bool packed_b = false,
                const ResidentCast* rc = nullptr, const SpecA* sp = nullptr) {
  if (M < 0 || N < 0 || K < 0 || K % 8 != 0 || N % 8 != 0 || K > kMaxK || N > kMaxN) return G16_E_SHAPE;
  if (M == 0 || N == 0) return G16_OK;
  if (ksplit < 1 || ksplit > 256) return G16_E_SPLIT;
  if (C == nullptr || (K > 0 && ((A == nullptr && rc == nullptr) || B == nullptr))) return G16_E_NULL;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return G16_E_ALIGN;
  const KSplit ks = ksplit_for(K, ksplit);
  if (num_cus <= 0) num_cus = stream_cus(static_cast<hipStream_t>(stream));
  Plan p = choose_tile(M, N, K, num_cus);
  if (rc != nullptr && !resident_route(p, ks.ksplit, K)) return G16_E_SHAPE;
  const bool spec = sp != nullptr;
  if (spec && (!four_wave(p.tile) || packed ||
               ks.ksplit > kSpecMaxSplit || sp->texp < kSpecMinTexp))
    return G16_E_SHAPE;
  if (packed) {
    // the packed layouts are the stage images of the 256-row tiles: the 256x256 tile, or the
    // 256x128 one where the plan picks it
    if (p.tile != Tile::T256N) p = Plan{Tile::T256, 256, 256, ceil_div(M, 256), ceil_div(N, 256)};
  }
  float* part = nullptr;
  uint32_t* counters = nullptr;
  if (ks.ksplit > 1) {
    if (ws == nullptr || ws_bytes < splitk_ws_bytes(p, ks.ksplit)) return G16_E_WORKSPACE;
    if (counters_in == nullptr || counter_bytes_in < splitk_counter_bytes(p, ks.ksplit)) return G16_E_WORKSPACE;
    if (!aligned16(ws) || !aligned16(counters_in)) return G16_E_ALIGN;
    counters = counters_in;
    part = static_cast<float*>(ws);
  }
  // The unsplit 256-row tiles hold one workgroup per CU: past one round, a persistent grid of one
  // workgroup per CU (a multiple of 8, so each keeps its XCD's tile range) walks the tiles.
  const bool big = p.tile == Tile::T256 || p.tile == Tile::T256N;
  const long ntiles = static_cast<long>(p.ntm) * p.ntn;
  const long persist = num_cus >= 8 ? num_cus / 8 * 8 : 8;
  const long gx = big && ks.ksplit == 1 && ntiles > persist ? persist : ntiles;
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(ks.ksplit)), block(big ? Cfg256::THREADS : 256);
  const auto* a = reinterpret_cast<const _Float16*>(A);
  const auto* b = reinterpret_cast<const _Float16*>(B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool sk = ks.ksplit > 1;
  const bool res = rc != nullptr;
  const void* x = res ? rc->x : nullptr;
  const int x_f32 = res ? rc->x_f32 : 0;
  const int texp = res ? rc->texp : (spec ? sp->texp : 0);
  const int tbits = spec ? sp->tbits : 0;
  uint32_t* miss = spec ? sp->miss : nullptr;
  if (out_f16)
    return launch(gemm_fn<true>(p.tile, sk, packed, packed_b, res, spec), grid, block, s, a, b, C, bias, rscale, part,
                  counters, M, N, K, ks.kchunk, ks.ksplit, p.ntm, p.ntn, x, x_f32, texp, tbits, miss);
  return launch(gemm_fn<false>(p.tile, sk, packed, packed_b, res, spec), grid, block, s, a, b, C, bias, rscale, part,
                counters, M, N, K, ks.kchunk, ks.ksplit, p.ntm, p.ntn, x, x_f32, texp, tbits, miss);
}

}  // namespace
}  // namespace g16

extern "C" int g16_hgemm_plan(int M, int N, int K, int num_cus) {
  // Split K when the output tiles leave CUs without a workgroup, into as many slices as keep the
  // grid within one workgroup per CU (the split-K kernels hold one workgroup per CU: a grid past
  // that runs a second round; 768 x 4096^2: 192 tiles unsplit 48 us, 2 slices 54 us;
  // 512 x 4096^2: 128 tiles unsplit 44 us, 2 slices 36 us; 512 x 11008 x 4096: 104 vs 75 us).
  if (M <= 0 || N <= 0 || K <= 0 || num_cus <= 0) return 1;
  const g16::Plan q = g16::choose_tile(M, N, K, num_cus);
  if (q.ks > 0) return q.ks;  // chosen with its tile (modelled_tile)
  const int tiles = q.ntm * q.ntn;
  if (tiles >= num_cus || K < g16::kMinSplitK) return 1;
  // At most 8 slices: the last slice to arrive reads every other slice's fp32 tile at one CU's
  // bandwidth, so beyond ~8 the reduction costs more than the extra parallelism gains (measured:
  // 64x4096x1024 12.1 us at 8 vs 14.3 us at 16). Each slice keeps >= 256 K (>= 1024 K for the
  // 128x128 tile, whose 64 KB partials make the reduction dearer; graph-timed: 1024^3 13.2 us
  // unsplit vs 14.3 at 2 slices, 1024 x 1024 x 2048 14.1 vs 17.2, but 1024 x 2048 x 1024 18.1 at 2
  // slices vs 21.1 unsplit and 20.2 at 4; 64x1024x1024 on the 64x128 tile is best at its K/256 cap,
  // 8.7 us at 4 vs 9.7 us at 2).
  int ks = num_cus / tiles;
  // The 256-row tiles keep >= 4096 K per slice: their 256 KB partials cost the exchange more than
  // idle CUs cost at shorter K (measured on 128 tiles of 256x256: 2048 x 4096 x 11008 202 us
  // unsplit, 184 us at 2 slices; 2048 x 4096^2 89.6 vs 89.7 us; 2048 x 2048 x 4096 53 vs 63 us).
  // choose_tile now gives those shapes 256x128 tiles that fill the CUs instead, so the planner
  // does not split the 256-row tiles; explicit splits (g16_hgemm_splitk) still run them.
  const bool big = q.tile == g16::Tile::T256 || q.tile == g16::Tile::T256N;
  const int cap = K / (big ? 4096 : (q.tile == g16::Tile::T128 ? 1024 : 256));
  ks = ks > cap ? cap : ks;
  ks = ks > 8 ? 8 : ks;
  return g16::ksplit_for(K, ks < 1 ? 1 : ks).ksplit;
}

extern "C" size_t g16_hgemm_splitk_workspace_bytes(int M, int N, int K, int ksplit, int num_cus) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const g16::KSplit ks = g16::ksplit_for(K, ksplit);
  const g16::Plan p = g16::choose_tile(M, N, K, num_cus > 0 ? num_cus : g16::current_cus());
  return g16::splitk_ws_bytes(p, ks.ksplit);
}

extern "C" size_t g16_hgemm_splitk_counter_bytes(int M, int N, int K, int ksplit, int num_cus) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const g16::KSplit ks = g16::ksplit_for(K, ksplit);
  const g16::Plan p = g16::choose_tile(M, N, K, num_cus > 0 ? num_cus : g16::current_cus());
  return g16::splitk_counter_bytes(p, ks.ksplit);
}

extern "C" int g16_hgemm_f32out(const uint16_t* A, const uint16_t* B, float* C, const float* bias, const float* rscale,
                                int M, int N, int K, void* stream) {
  return g16::gemm_launch(A, B, C, false, bias, rscale, M, N, K, 1, 0, nullptr, 0, nullptr, 0, stream);
}

extern "C" int g16_hgemm_f16out(const uint16_t* A, const uint16_t* B, uint16_t* C, const float* bias,
                                const float* rscale, int M, int N, int K, void* stream) {
  return g16::gemm_launch(A, B, C, true, bias, rscale, M, N, K, 1, 0, nullptr, 0, nullptr, 0, stream);
}

extern "C" int g16_hgemm_use_packed(int M, int N, int K, int num_cus) {
  // The packed route pays off where the plain plan already picks the 256x256 tile without a split.
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const g16::Tile t = g16::choose_tile(M, N, K, num_cus).tile;
  return (t == g16::Tile::T256 || t == g16::Tile::T256N) && g16_hgemm_plan(M, N, K, num_cus) == 1 ? 1 : 0;
}

extern "C" int g16_hgemm_tile(int M, int N, int K, int num_cus, int* rows, int* cols) {
  // the tile choose_tile() plans: the one the launches, g16_hgemm_plan and the size queries use
  if (rows == nullptr || cols == nullptr) return G16_E_NULL;
  if (M <= 0 || N <= 0 || K <= 0) return G16_E_SHAPE;
  const g16::Plan p = g16::choose_tile(M, N, K, num_cus > 0 ? num_cus : g16::current_cus());
  *rows = p.bm;
  *cols = p.bn;
  return G16_OK;
}

extern "C" int g16_hgemm_use_packed_b(int M, int N, int K, int num_cus) {
  // A prepacked weight (g16_pack_weight) holds the B stage images of both 256-row tiles (whole
  // blocks for 256 columns, half blocks for 128), so it serves the whole packed route.
  return g16_hgemm_use_packed(M, N, K, num_cus);
}

extern "C" int g16_hgemm_packed_f32out(const uint16_t* Ap, const uint16_t* B, float* C, const float* bias,
                                      const float* rscale, int M, int N, int K, void* stream) {
  return g16::gemm_launch(Ap, B, C, false, bias, rscale, M, N, K, 1, 0, nullptr, 0, nullptr, 0, stream, true);
}

extern "C" int g16_hgemm_packed_f16out(const uint16_t* Ap, const uint16_t* B, uint16_t* C, const float* bias,
                                      const float* rscale, int M, int N, int K, void* stream) {
  return g16::gemm_launch(Ap, B, C, true, bias, rscale, M, N, K, 1, 0, nullptr, 0, nullptr, 0, stream, true);
}

extern "C" int g16_hgemm_packed_ab_f32out(const uint16_t* Ap, const uint16_t* Bp, float* C, const float* bias,
                                         const float* rscale, int M, int N, int K, void* stream) {
  return g16::gemm_launch(Ap, Bp, C, false, bias, rscale, M, N, K, 1, 0, nullptr, 0, nullptr, 0, stream, true, true);
}

extern "C" int g16_hgemm_packed_ab_f16out(const uint16_t* Ap, const uint16_t* Bp, uint16_t* C, const float* bias,
                                         const float* rscale, int M, int N, int K, void* stream) {
  return g16::gemm_launch(Ap, Bp, C, true, bias, rscale, M, N, K, 1, 0, nullptr, 0, nullptr, 0, stream, true, true);
}

extern "C" int g16_hgemm_splitk(const uint16_t* A, const uint16_t* B, void* C, int c_is_f16, const float* bias,
                                const float* rscale, int M, int N, int K, int ksplit, int num_cus, void* workspace,
                                size_t workspace_bytes, uint32_t* counters, size_t counter_bytes, void* stream) {
  return g16::gemm_launch(A, B, C, c_is_f16 != 0, bias, rscale, M, N, K, ksplit, num_cus, workspace, workspace_bytes,
                          counters, counter_bytes, stream);
}

namespace g16 {
namespace {

// The fp16 cast and the row scales share one scratch buffer: [cast, padded to 256 bytes][M floats].
size_t cast_bytes(int M, int K, bool packed) {
  return packed ? packed_bytes_for(M, K) : static_cast<size_t>(M) * K * 2;
}
size_t round256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace
}  // namespace g16

namespace g16 {
namespace {

bool mm_t_resident(int M, int N, int K, int num_cus) {
  if (M <= 0 || N <= 0 || K <= 0 || num_cus <= 0 || g16_hgemm_use_packed(M, N, K, num_cus) == 1) return false;
  return resident_route(choose_tile(M, N, K, num_cus), ksplit_for(K, g16_hgemm_plan(M, N, K, num_cus)).ksplit, K);
}

// Speculation history, per device, once g16_mm_t_spec_history has enabled it: a speculative launch
// that had to compute a tile again stores 1 into its weight's slot (pinned host memory, written by
// the kernel). g16_mm_t_gemm then sends the weight's next kSpecRetry - 1 calls down the resident or
// two-launch route (the same result bits, without the recomputation) and speculates again after
// that. Weights whose pointers hash alike share a slot; the route never changes a result, only its
// time.
constexpr int kSpecSlots = 1024;
constexpr uint32_t kSpecRetry = 64;
struct SpecHistory {
  uint32_t* miss = nullptr;                  // kSpecSlots words (hipHostMalloc, never freed)
  std::atomic<uint32_t> routed[kSpecSlots];  // calls routed around speculation since the slot's miss
};

size_t spec_slot(const void* w_t) {
  const uint64_t h = (static_cast<uint64_t>(reinterpret_cast<uintptr_t>(w_t)) >> 8) * 0x9e3779b97f4a7c15ull;
  return static_cast<size_t>(h >> 54);  // top 10 bits: kSpecSlots
}
static_assert(kSpecSlots == 1024, "spec_slot keeps 10 bits");

// The histories, per device, once g16_mm_t_spec_history has allocated them (the GEMM entry points
// themselves never allocate).
std::atomic<SpecHistory*> g_spec_hist[64];
std::mutex g_spec_mu;

int stream_device(hipStream_t stream) {
  int dev = 0;
  if (stream == nullptr || hipStreamGetDevice(stream, &dev) != hipSuccess) {
    if (hipGetDevice(&dev) != hipSuccess) return -1;
  }
  return dev >= 0 && dev < 64 ? dev : -1;
}

// The history of the device that owns `stream`, or NULL if it has none.
SpecHistory* spec_history(hipStream_t stream) {
  const int dev = stream_device(stream);
  return dev < 0 ? nullptr : g_spec_hist[dev].load(std::memory_order_acquire);
}

// fp16 x runs as one speculative launch wherever the plan is a 4-wavefront tile.
bool mm_t_speculative(int M, int N, int K, int num_cus) {
  if (M <= 0 || N <= 0 || K <= 0 || num_cus <= 0 || g16_hgemm_use_packed(M, N, K, num_cus) == 1) return false;
  const Tile t = choose_tile(M, N, K, num_cus).tile;
  return four_wave(t);
}

}  // namespace
}  // namespace g16

extern "C" size_t g16_mm_t_scratch_bytes(int M, int N, int K, int num_cus) {
  if (M <= 0 || N <= 0 || K < 0) return 0;
  if (g16::mm_t_resident(M, N, K, num_cus)) return 0;  // one launch; the cast stays in LDS
  const bool packed = g16_hgemm_use_packed(M, N, K, num_cus) == 1;
  return g16::round256(g16::cast_bytes(M, K, packed)) + static_cast<size_t>(M) * sizeof(float);
}

extern "C" int g16_mm_t_gemm(const void* x, int x_is_f32, const uint16_t* w_t, void* out, int out_is_f16,
                             const float* bias, float thresh, int M, int N, int K, int num_cus, void* scratch,
                             size_t scratch_bytes, void* workspace, size_t workspace_bytes, uint32_t* counters,
                             size_t counter_bytes, void* stream) {
  // mm_t's GEMM path in one call: the same two launches, and the same result bits, as the
  // separate rowscale and GEMM entry points on the route g16_hgemm_use_packed / g16_hgemm_plan pick
  if (M < 0 || N < 0 || K < 0 || K % 8 != 0 || N % 8 != 0 || K > g16::kMaxK || N > g16::kMaxN || num_cus <= 0)
    return G16_E_SHAPE;
  if (M == 0 || N == 0) return G16_OK;
  if (out == nullptr || (K > 0 && (x == nullptr || w_t == nullptr))) return G16_E_NULL;
  const int texp = g16::thresh_exponent(thresh);
  if (texp == -1000) return G16_E_SHAPE;
  if (!x_is_f32 && texp >= g16::kSpecMinTexp && g16::mm_t_speculative(M, N, K, num_cus)) {
    // fp16 x on the 4-wavefront tiles: one launch that streams x as A (a row within the threshold
    // is its own cast) and computes a tile again, with A rescaled in registers, only where some
    // |x| exceeds it; no scratch. Where the caller's scratch allows the other route, a weight
    // whose recent call was computed again takes that route for a while instead.
    const bool other_route =
        g16::mm_t_resident(M, N, K, num_cus) ||
        (scratch != nullptr && g16::aligned16(scratch) && scratch_bytes >= g16_mm_t_scratch_bytes(M, N, K, num_cus));
    bool speculate = true;
    uint32_t* miss = nullptr;
    if (other_route) {
      if (g16::SpecHistory* h = g16::spec_history(static_cast<hipStream_t>(stream))) {
        const size_t slot = g16::spec_slot(w_t);
        miss = h->miss + slot;
        if (__atomic_load_n(miss, __ATOMIC_RELAXED) != 0u) {
          if (h->routed[slot].fetch_add(1, std::memory_order_relaxed) + 1 < g16::kSpecRetry) {
            speculate = false;
          } else {
            h->routed[slot].store(0, std::memory_order_relaxed);
            __atomic_store_n(miss, 0u, __ATOMIC_RELAXED);
          }
        }
      }
    }
    if (speculate) {
      const g16::SpecA sp{texp, g16::fp16_bits_at_most(texp), miss};
      const int ks = g16_hgemm_plan(M, N, K, num_cus);
      return g16::gemm_launch(static_cast<const uint16_t*>(x), w_t, out, out_is_f16 != 0, bias, nullptr, M, N, K, ks,
                              num_cus, workspace, workspace_bytes, counters, counter_bytes, stream, false, false,
                              nullptr, &sp);
    }
  }
  if (g16::mm_t_resident(M, N, K, num_cus)) {
    // one launch: the GEMM's workgroups cast their own rows into LDS (the same bits as the cast
    // below, the same GEMM arithmetic); no scratch
    if (!g16::aligned16(x)) return G16_E_ALIGN;
    const g16::ResidentCast rc{x, x_is_f32 != 0 ? 1 : 0, texp};
    return g16::gemm_launch(nullptr, w_t, out, out_is_f16 != 0, bias, nullptr, M, N, K, 1, num_cus, nullptr, 0, nullptr,
                            0, stream, false, false, &rc);
  }
  if (scratch == nullptr) return G16_E_NULL;
  if (!g16::aligned16(scratch)) return G16_E_ALIGN;
  if (scratch_bytes < g16_mm_t_scratch_bytes(M, N, K, num_cus)) return G16_E_WORKSPACE;
  const bool packed = g16_hgemm_use_packed(M, N, K, num_cus) == 1;
  auto* y = static_cast<uint16_t*>(scratch);
  auto* s = reinterpret_cast<float*>(static_cast<unsigned char*>(scratch) + g16::round256(g16::cast_bytes(M, K, packed)));
  int st;
  if (x_is_f32)
    st = packed ? g16_rowscale_pack_f32(static_cast<const float*>(x), y, s, M, K, thresh, stream)
                : g16_rowscale_f32(static_cast<const float*>(x), y, s, M, K, thresh, stream);
  else
    st = packed ? g16_rowscale_pack_f16(static_cast<const uint16_t*>(x), y, s, M, K, thresh, stream)
                : g16_rowscale_f16(static_cast<const uint16_t*>(x), y, s, M, K, thresh, stream);
  if (st != G16_OK) return st;
  if (packed)
    return g16::gemm_launch(y, w_t, out, out_is_f16 != 0, bias, s, M, N, K, 1, num_cus, nullptr, 0, nullptr, 0, stream,
                            true);
  const int ks = g16_hgemm_plan(M, N, K, num_cus);
  return g16::gemm_launch(y, w_t, out, out_is_f16 != 0, bias, s, M, N, K, ks, num_cus, workspace, workspace_bytes,
                          counters, counter_bytes, stream);
}

extern "C" int g16_mm_t_spec_history(void* stream) {
  // once per device: the pinned words the speculative launches report recomputations into
  const int dev = g16::stream_device(static_cast<hipStream_t>(stream));
  if (dev < 0) return G16_E_NULL;
  if (g16::g_spec_hist[dev].load(std::memory_order_acquire) != nullptr) return G16_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (stream != nullptr) {
    const hipError_t e = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cap);
    if (e != hipSuccess) return static_cast<int>(e);
    if (cap != hipStreamCaptureStatusNone) return static_cast<int>(hipErrorStreamCaptureUnsupported);
  }
  std::lock_guard<std::mutex> lock(g16::g_spec_mu);
  if (g16::g_spec_hist[dev].load(std::memory_order_acquire) != nullptr) return G16_OK;
  g16::StreamDeviceScope on_device(static_cast<hipStream_t>(stream));
  void* p = nullptr;
  const hipError_t e = hipHostMalloc(&p, g16::kSpecSlots * sizeof(uint32_t), hipHostMallocPortable | hipHostMallocCoherent);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // reported here; leave no sticky error behind
    return static_cast<int>(e);
  }
  __builtin_memset(p, 0, g16::kSpecSlots * sizeof(uint32_t));
  auto* h = new g16::SpecHistory;
  h->miss = static_cast<uint32_t*>(p);
  for (auto& r : h->routed) r.store(0, std::memory_order_relaxed);
  g16::g_spec_hist[dev].store(h, std::memory_order_release);
  return G16_OK;
}

extern "C" int g16_mm_t_spec_paused(const uint16_t* w_t, void* stream) {
  const g16::SpecHistory* h = g16::spec_history(static_cast<hipStream_t>(stream));
  return h != nullptr && __atomic_load_n(h->miss + g16::spec_slot(w_t), __ATOMIC_RELAXED) != 0u ? 1 : 0;
}

extern "C" int g16_gemm_clock(unsigned long long* dst, void* stream) {
  // ordered after the GEMMs already enqueued on `stream`: their stamps are final when it runs
  if (dst == nullptr) return G16_E_NULL;
  if ((reinterpret_cast<uintptr_t>(dst) & 7u) != 0) return G16_E_ALIGN;
  return g16::launch(g16::copy_loop_clock, dim3(1), dim3(1), static_cast<hipStream_t>(stream), dst);
}
