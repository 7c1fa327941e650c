/*
 * g16.h -- C ABI of libg16.so, the gfx950 (MI355X) kernels behind gtx16_fp16.mm_t / matmul /
 * FastLinear.
 *
 * Each entry point replaces one kernel that the reference compiles with NVRTC and launches by name
 * through cuLaunchKernel (src/gtx16_fp16/kernels.py:282-338). Paths below are relative to the
 * reference checkout.
 *
 * Conventions shared by every entry point:
 *   - Plain device pointers and sizes; no torch types. fp16 data is passed as uint16_t bit
 *     patterns (IEEE binary16), fp32 as float.
 *   - The call enqueues work on `stream` (a hipStream_t; NULL = the legacy default stream of the
 *     current device) and returns at once. The kernels run on the device that owns `stream`: when
 *     that is not the calling thread's current device, the call makes it current for the launch
 *     and restores the previous one. It never synchronises and never allocates or frees device
 *     memory.
 *   - Return value: 0 on success; a negative G16_E* code for an argument the library rejects
 *     (nothing is enqueued then); a positive hipError_t if the HIP launch itself fails.
 *     g16_strerror() names both kinds.
 *   - Row-major, contiguous operands: x/A is [M,K], the weight w_t/B is [K,N] (N contiguous),
 *     outputs are [M,N]. K and N must be multiples of 8 and every pointer 16-byte aligned (the
 *     reference's supported() predicate, src/gtx16_fp16/ops.py:29-35, plus the alignment the
 *     16-byte vector loads need). M == 0 or N == 0 is a no-op. The GEMM entry points (hgemm_*,
 *     mm_t_gemm) also need K <= G16_GEMM_MAX_K and N <= G16_GEMM_MAX_N (their operands are
 *     addressed through 32-bit buffer offsets) and return G16_E_SHAPE beyond them.
 *   - num_cus: where an entry point plans its launch for a compute-unit count, the GEMM tile and
 *     hence the split buffers' sizes follow that count. A caller that plans ksplit and sizes the
 *     split buffers for one count must launch with the same count; num_cus <= 0 means the device's
 *     own count (the stream's device for a launch, the current device for a size query).
 *   - Split reductions (split-K and skinny paths) take two caller-owned device buffers:
 *       workspace -- fp32 partial sums, at least *_workspace_bytes(); needs no initialisation;
 *       counters  -- per-tile arrival counters, at least *_counter_bytes(); must be all zero
 *                    before the first use, and every call leaves them all zero again, so one
 *                    zero-filled counter buffer serves any sequence of calls on one stream.
 *     With ksplit == 1 neither is used (NULL/0 is fine). Calls that use the same buffers
 *     concurrently (different streams) race.
 *   - Results are deterministic: no floating-point atomics; split reductions sum partials in a
 *     fixed order, so repeated calls return identical bits.
 */
#ifndef G16_H
#define G16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G16_ABI_VERSION 16

/* Status codes (negative: rejected by the library before any launch). */
#define G16_OK 0
#define G16_E_SHAPE (-1)       /* negative size, K or N not a multiple of 8, or a GEMM K or N past its limit */
#define G16_E_ALIGN (-2)       /* a pointer is not 16-byte aligned */
#define G16_E_NULL (-3)        /* a required pointer is NULL */
#define G16_E_WORKSPACE (-4)   /* workspace or counters missing or smaller than required */
#define G16_E_SPLIT (-5)       /* ksplit out of range */
#define G16_E_DTYPE (-6)       /* unknown dtype code */
#define G16_E_TOO_LARGE (-7)   /* the split does not fit the static scratch of a _noalloc entry point */

/* Size limits of the GEMM entry points (32-bit DMA offsets; see above). */
#define G16_GEMM_MAX_K ((1 << 22) - 8)
#define G16_GEMM_MAX_N ((1 << 24) - 8)

/* Semantic constants of the reference. */
#define G16_SKINNY_MAX_M 8          /* src/gtx16_fp16/kernels.py:253 */
#define G16_ROW_SCALE_THRESHOLD 1024.0f /* src/gtx16_fp16/ops.py:16 */

int g16_abi_version(void);
const char* g16_strerror(int status);

/* ---------------------------------------------------------------------------------------------
 * Row rescale + fp16 cast.
 * Replaces rowscale_f32 / rowscale_f16 (src/gtx16_fp16/kernels.py:227-250), launched at
 * src/gtx16_fp16/ops.py:86-90 with grid (M,1,1) -- here M is an argument.
 * Per row i: amax = max_k |X[i,k]| (NaN ignored); S[i] = 2^ceil(log2(amax/thresh)) when
 * amax > thresh, else 1 (+inf for an infinite row); Y[i,k] = fp16_rne(X[i,k] / S[i]).
 * thresh must be a positive power of two (the reference uses 1024).
 */
int g16_rowscale_f32(const float* X, uint16_t* Y, float* S, int M, int K, float thresh,
                     void* stream);
int g16_rowscale_f16(const uint16_t* X, uint16_t* Y, float* S, int M, int K, float thresh,
                     void* stream);

/* ---------------------------------------------------------------------------------------------
 * Tiled MFMA GEMM: C[M,N] = rscale[row] * (A16[M,K] @ B16[K,N]) + bias[N], fp32 accumulation.
 * Replaces hgemm_f32out / hgemm_f16out (src/gtx16_fp16/kernels.py:139-142,148-151), launched at
 * src/gtx16_fp16/ops.py:103-108. bias and rscale may be NULL (0 and 1). fp16 output rounds to
 * nearest-even.
 */
int g16_hgemm_f32out(const uint16_t* A, const uint16_t* B, float* C, const float* bias,
                     const float* rscale, int M, int N, int K, void* stream);
int g16_hgemm_f16out(const uint16_t* A, const uint16_t* B, uint16_t* C, const float* bias,
                     const float* rscale, int M, int N, int K, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Tile-packed route for the large GEMM: the same two reference kernels as above, rowscale_f32 /
 * rowscale_f16 (src/gtx16_fp16/kernels.py:227-250) then hgemm_f32out / hgemm_f16out
 * (kernels.py:139-142,148-151), as launched by src/gtx16_fp16/ops.py:86-90,103-108, with the fp16
 * intermediate written in a layout the 256-row GEMM tiles (256x256, and 256x128 where the plan
 * picks it) stream as contiguous 16 KB blocks instead of row-major. Same values, same results bit
 * for bit; only the intermediate's layout differs.
 *   Packed layout of Yp: blocks of 256 rows x 32 columns, block (tm, ks) at block index
 *   tm * ceil(K/32) + ks, 16 KB each; inside a block, 16-byte chunk q*64 + i (q < 16, i < 64)
 *   holds columns 8*((i % 4) ^ ((r / 2) % 4)) .. +7 of local row r = 16q + i/4. Rows >= M and
 *   columns >= K are written as zeros. g16_packed_a_bytes() gives the size.
 * g16_hgemm_use_packed() is 1 where mm_t takes this route (the plain plan would use a 256-row tile
 * without a split), else 0. The packed GEMM accepts any shape.
 */
size_t g16_packed_a_bytes(int M, int K);
int g16_rowscale_pack_f32(const float* X, uint16_t* Yp, float* S, int M, int K, float thresh,
                          void* stream);
int g16_rowscale_pack_f16(const uint16_t* X, uint16_t* Yp, float* S, int M, int K, float thresh,
                          void* stream);
int g16_hgemm_packed_f32out(const uint16_t* Ap, const uint16_t* B, float* C, const float* bias,
                            const float* rscale, int M, int N, int K, void* stream);
int g16_hgemm_packed_f16out(const uint16_t* Ap, const uint16_t* B, uint16_t* C, const float* bias,
                            const float* rscale, int M, int N, int K, void* stream);
int g16_hgemm_use_packed(int M, int N, int K, int num_cus);

/* ---------------------------------------------------------------------------------------------
 * mm_t's GEMM path (src/gtx16_fp16/ops.py:86-108) in one call: the rowscale cast of x (fp32 when
 * x_is_f32, else fp16) into `scratch`, then the GEMM on the route this library plans for num_cus
 * compute units -- the tile-packed route where g16_hgemm_use_packed() is 1, else split-K with
 * ksplit = g16_hgemm_plan() when that is > 1, else the plain GEMM. The same result bits as the
 * separate entry points (rowscale, then GEMM); one call instead of two on a path whose small
 * shapes are bound by host and launch time. No counterpart kernel in the reference.
 *   One launch for fp16 x where the plan is a 4-wavefront tile (32x128, 64x128, 64x64 or
 *   128x128, split or not) and thresh >= 2^-8: the GEMM streams x itself as A, since a row within
 *   the threshold is its own cast, and computes a tile again, with A rescaled in registers by the
 *   rows' exponents, only where some |x| of it exceeds the threshold or is NaN (split tiles: the
 *   last slice to arrive recomputes every slice). Same result bits; no scratch is used. A weight whose call had
 *   a tile computed again takes the other route below for its next 63 calls when the scratch the
 *   caller passed allows it (a per-device history in pinned host memory, keyed by w_t, once
 *   g16_mm_t_spec_history has enabled it).
 *   One launch for fp32 x where the plan is the unsplit 32x128 tile and K <= 1280: the GEMM's
 *   workgroups cast their own rows of x into LDS (the rowscale arithmetic, the same bits) and no
 *   rowscale launch runs; g16_mm_t_scratch_bytes() is then 0 and scratch may be NULL (x must be
 *   16-byte aligned). Elsewhere the call makes the two launches.
 *   scratch: at least g16_mm_t_scratch_bytes(M, N, K, num_cus) bytes, 16-byte aligned (the fp16
 *   cast and the row scales; it must stay allocated until the GEMM has run). It may be NULL on the
 *   one-launch routes above (fp16 x then always takes the one launch).
 *   workspace / counters: as g16_hgemm_splitk needs them for that ksplit (unused otherwise, then
 *   NULL/0 is fine). thresh: as for the rowscale entry points.
 */
size_t g16_mm_t_scratch_bytes(int M, int N, int K, int num_cus);
int g16_mm_t_gemm(const void* x, int x_is_f32, const uint16_t* w_t, void* out, int out_is_f16,
                  const float* bias, float thresh, int M, int N, int K, int num_cus, void* scratch,
                  size_t scratch_bytes, void* workspace, size_t workspace_bytes, uint32_t* counters,
                  size_t counter_bytes, void* stream);
/* Enables the speculation history for the device that owns `stream` (no counterpart in the
 * reference): allocates 4 KB of pinned host memory once per device (kept until the process ends)
 * into which the one-launch fp16 kernels report a recomputation. Until it is called,
 * g16_mm_t_gemm keeps the one-launch route for every call. Returns 0, or the HIP error of the
 * allocation (hipErrorStreamCaptureUnsupported while `stream` is being captured). Thread-safe;
 * later calls return 0 at once. The GEMM entry points themselves never allocate. */
int g16_mm_t_spec_history(void* stream);
/* 1 if the speculation history of the device that owns `stream` routes g16_mm_t_gemm's next call
 * with this w_t around the one-launch fp16 route (a recent call with it was computed again), else
 * 0 (also when the history is not enabled). For tests and diagnostics; no counterpart in the
 * reference. */
int g16_mm_t_spec_paused(const uint16_t* w_t, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Prepacked weight for the large GEMM (no counterpart kernel in the reference; it serves
 * FastLinear, src/gtx16_fp16/linear.py:12-76, whose fp16 weight_t [K,N] is fixed after from_linear,
 * linear.py:30-37). g16_pack_weight writes w_t transposed ([N,K]) in the tile-packed layout above
 * (rows = N); g16_hgemm_packed_ab_* is the packed GEMM with both operands packed. Same values and
 * the same result bits as g16_hgemm_packed_* on the unpacked weight.
 * g16_hgemm_use_packed_b() is 1 where a packed weight serves mm_t's route: the packed route, on
 * either 256-row tile (the 256x128 tile streams half blocks of the same layout).
 */
size_t g16_packed_b_bytes(int K, int N);
int g16_pack_weight(const uint16_t* w_t, uint16_t* wp, int K, int N, void* stream);
int g16_hgemm_packed_ab_f32out(const uint16_t* Ap, const uint16_t* Bp, float* C, const float* bias,
                               const float* rscale, int M, int N, int K, void* stream);
int g16_hgemm_packed_ab_f16out(const uint16_t* Ap, const uint16_t* Bp, uint16_t* C,
                               const float* bias, const float* rscale, int M, int N, int K,
                               void* stream);
int g16_hgemm_use_packed_b(int M, int N, int K, int num_cus);

/* ---------------------------------------------------------------------------------------------
 * Deterministic split-K GEMM for shapes with too few output tiles to fill the GPU.
 * Replaces hgemm_splitk + the bias prefill _prefilled (src/gtx16_fp16/kernels.py:143-147,
 * src/gtx16_fp16/ops.py:54-62,92-101). Instead of fp32 atomics into a prefilled C, each K slice
 * writes an fp32 partial tile to the workspace; the last slice to finish a tile sums the partials
 * in slice order, then applies rscale and bias and writes C (fp32, or fp16 when c_is_f16 != 0,
 * so no separate cast pass). ksplit in [1, 256]; ksplit == 1 needs no workspace.
 * g16_hgemm_plan() returns the ksplit this library would choose (1 = the plain GEMM). The tile the
 * launch runs on, and so the workspace and counter sizes, depend on num_cus (see above): pass the
 * same num_cus to the plan, the two size queries and the launch.
 */
int g16_hgemm_splitk(const uint16_t* A, const uint16_t* B, void* C, int c_is_f16,
                     const float* bias, const float* rscale, int M, int N, int K, int ksplit,
                     int num_cus, void* workspace, size_t workspace_bytes, uint32_t* counters,
                     size_t counter_bytes, void* stream);
size_t g16_hgemm_splitk_workspace_bytes(int M, int N, int K, int ksplit, int num_cus);
size_t g16_hgemm_splitk_counter_bytes(int M, int N, int K, int ksplit, int num_cus);
int g16_hgemm_plan(int M, int N, int K, int num_cus);
/* The tile the GEMM entry points run (M, N, K) on for num_cus compute units (<= 0: the current
 * device's): *rows x *cols is 32x128, 64x128, 64x64 or 128x128 (4 wavefronts), 256x128 or 256x256
 * (8 wavefronts; the tile-packed route). The plan above and the split-buffer sizes are for this
 * tile. No counterpart in the reference (its GEMM has one 128x128 tile); for tests and
 * diagnostics. Returns G16_E_SHAPE for M, N or K <= 0. */
int g16_hgemm_tile(int M, int N, int K, int num_cus, int* rows, int* cols);

/* ---------------------------------------------------------------------------------------------
 * Skinny GEMM (GEMV-like) for 1 <= M <= 8: C[M,N] = A[M,K] @ B16[K,N] + bias, fp32 math on the
 * UNQUANTISED activations (fp32 or fp16), fp32 output.
 * Replaces skinny_f32in / skinny_f16in (src/gtx16_fp16/kernels.py:212-219) and its launch
 * configuration skinny_config (src/gtx16_fp16/ops.py:45-51,78-84; src/gtx16_fp16/linear.py:49-64).
 * A is read with 16-byte alignment (A must be 16-byte aligned, like B).
 * The kernel streams B once with 16-byte loads; K is split over ksplit workgroups per strip of
 * g16_skinny_strip_cols(M, N) columns (256 up to N = 8192, 512 above) and reduced
 * deterministically (last arriving workgroup, slice order). C needs no zero-fill.
 * The split workspace (ksplit * M * N * 4 bytes) must stay below 2 GiB (G16_E_SPLIT otherwise).
 * g16_skinny_plan() returns the ksplit this library would choose for num_cus compute units; the
 * launch grid is ceil(N / strip columns) * ksplit workgroups of 512 threads.
 */
int g16_skinny_f32in(const float* A, const uint16_t* B, float* C, const float* bias, int M, int N,
                     int K, int ksplit, void* workspace, size_t workspace_bytes, uint32_t* counters,
                     size_t counter_bytes, void* stream);
int g16_skinny_f16in(const uint16_t* A, const uint16_t* B, float* C, const float* bias, int M,
                     int N, int K, int ksplit, void* workspace, size_t workspace_bytes,
                     uint32_t* counters, size_t counter_bytes, void* stream);
size_t g16_skinny_workspace_bytes(int M, int N, int K, int ksplit);
size_t g16_skinny_counter_bytes(int M, int N, int K, int ksplit);
int g16_skinny_plan(int M, int N, int K, int num_cus);
int g16_skinny_strip_cols(int M, int N);

/* g16_skinny_f32in without caller buffers and without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight decode/serving loops, harnesses that forbid hipMalloc). Same arguments, kernels and result
 * bits as g16_skinny_f32in minus the four buffer arguments: the split partials and arrival
 * counters live in a static device array the library holds on every GPU it runs on until the
 * process ends (G16_NOALLOC_PARTIAL_BYTES of partials, G16_NOALLOC_COUNTER_BYTES of counters:
 * ksplit * M * N * 4 <= 4 MiB and N <= 131072). A split that does not fit returns
 * G16_E_TOO_LARGE before any launch; use g16_skinny_f32in with your own buffers then. The first
 * call on a device also enqueues a small kernel that zeroes the counters. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other threads) race. */
#define G16_NOALLOC_PARTIAL_BYTES (4 << 20)
#define G16_NOALLOC_COUNTER_BYTES (64 << 10)
int g16_skinny_f32in_noalloc(const float* A, const uint16_t* B, float* C, const float* bias, int M,
                             int N, int K, int ksplit, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Skinny GEMM on FastLinear's decode layout (no counterpart kernel in the reference; it serves the
 * token-by-token branch of FastLinear.forward, src/gtx16_fp16/linear.py:49-64, whose fp16 weight_t
 * [K,N] is fixed after from_linear, linear.py:30-37). Same semantics as g16_skinny_f32in /
 * g16_skinny_f16in for 1 <= M <= G16_STRIPS_MAX_M: C[M,N] = A[M,K] @ B16[K,N] + bias in fp32 on
 * the unquantised activations, fp32 output.
 * g16_pack_decode_weight writes w_t [K,N] as N/8 strips of 8 columns, each strip all K rows long
 * and contiguous: wd[(s*K + k)*8 + c] = w_t[k*N + 8*s + c] (K*N fp16 elements, like w_t).
 * g16_skinny_strips_* run one workgroup of 512 threads per strip over all of K: no split, no
 * workspace, no counters, C needs no zero-fill, and the result is bitwise reproducible (it differs
 * from g16_skinny_* in the order of the fp32 additions only). A, wd and C 16-byte aligned;
 * K and N multiples of 8.
 */
#define G16_STRIPS_MAX_M 4
int g16_pack_decode_weight(const uint16_t* w_t, uint16_t* wd, int K, int N, void* stream);
int g16_skinny_strips_f32in(const float* A, const uint16_t* wd, float* C, const float* bias, int M,
                            int N, int K, void* stream);
int g16_skinny_strips_f16in(const uint16_t* A, const uint16_t* wd, float* C, const float* bias,
                            int M, int N, int K, void* stream);
/* 1 where g16_skinny_strips_* is expected to be faster than g16_skinny_* for this product (a
 * measured rule: M <= 2, or small weights, or fp16 activations at M = 3 and at M = 4 up to
 * N = 8192); 0 otherwise or for sizes out of range. x_f32: 1 for fp32 activations, 0 for fp16. */
int g16_skinny_strips_route(int M, int N, int K, int x_f32);

/* ---------------------------------------------------------------------------------------------
 * Clock of the latest GEMM launch (no counterpart in the reference; a measurement aid for the
 * benchmark, whose rooflines depend on the clock a power-limited part holds). Every hgemm launch
 * (any route) has its workgroup 0 record the shader cycles and the 100 MHz reference ticks its main
 * loop took; g16_gemm_clock enqueues on `stream` a copy of the latest launch's pair into dst[0]
 * (cycles) and dst[1] (ticks), device memory, 8-byte aligned. Clock in MHz: 100 * dst[0] / dst[1].
 * Launches on other streams of the device race for the same record.
 */
int g16_gemm_clock(unsigned long long* dst, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Peak microbenchmark: the MI355X counterpart of the reference's bench/peak.py:1-63 (which times
 * FFMA, HFMA2 and mma.sync kernels). No counterpart in the kernel ABI: it measures the instruction
 * and bandwidth peaks the benchmark's rooflines divide by, at the clocks the part holds.
 * kind 0: fp32 FMA (VALU); 1: packed fp16 FMA; 2: MFMA 32x32x16 f16; 3: MFMA 16x16x32 f16;
 * 4, 5: kinds 2, 3 on random fp16 operand bits (the MFMA power, hence the clock the part holds,
 * depends on operand toggling: 2 and 3 run at the top clock, 4 and 5 at the clock real data gets);
 * 6: LDS reads with ds_read_b128; 7: LDS transposing reads with ds_read_b64_tr_b16 (32 KB of LDS
 * per workgroup, so at most five workgroups share a CU).
 * g16_peak_run launches `blocks` workgroups of 256 lanes looping `iters` times; each lane does
 * g16_peak_flops_per_lane_iter(kind) flops (kinds 0-5) or LDS bytes (kinds 6, 7) per iteration.
 * `out` holds blocks * 256 floats.
 * g16_peak_run_clocked does the same and, when `clocks` is not NULL, stores into clocks[0] the
 * shader clock cycles and into clocks[1] the 100 MHz reference ticks of workgroup 0's loop.
 * g16_stream_read reads `bytes` (a multiple of 16, 16-byte aligned buffer) once with 16-byte
 * loads from `blocks` workgroups of 256 lanes; `out` holds blocks * 256 floats.
 * g16_peak_mfma_data (kind 8 of g16_peak_flops_per_lane_iter) runs the 256x256 GEMM tile's per-
 * wavefront MFMA stream (8 A x 4 B fragments, 32 v_mfma_f32_16x16x32_f16 per step in the tile's
 * snake order, two fragment sets alternating per step) on caller-supplied operands, `iters`
 * iterations of two steps, from `blocks` workgroups of 256 lanes. `operands` (16-byte aligned)
 * holds ngroups * 256 * 24 fragments of 8 fp16 values: fragment f (0-7 A, 8-11 B) of set s for
 * lane t of workgroup b is operands[(((b % ngroups) * 256 + t) * 2 + s) * 12 + f]. `out`
 * (16-byte aligned) receives blocks * 256 * 128 floats: lane t of workgroup b stores accumulator
 * (i, j) register r at out[(b * 256 + t) * 128 + (4 i + j) * 4 + r]. `clocks` as above.
 */
double g16_peak_flops_per_lane_iter(int kind);
int g16_peak_run(int kind, int blocks, int iters, float* out, void* stream);
int g16_peak_run_clocked(int kind, int blocks, int iters, float* out, unsigned long long* clocks, void* stream);
int g16_stream_read(const void* buf, size_t bytes, int blocks, float* out, void* stream);
int g16_peak_mfma_data(int blocks, int iters, const uint16_t* operands, int ngroups, float* out,
                       unsigned long long* clocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* G16_H */
