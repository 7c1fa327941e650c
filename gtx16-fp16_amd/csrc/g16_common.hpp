// Shared helpers for the gfx950 kernels of libg16.so: vector types, launch wrapper, argument
// checks, and the cross-workgroup "last arrival" handshake used by the deterministic split
// reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "g16.h"

namespace g16 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

template <typename T>
struct identity {
  using type = T;
};

// Makes the device that owns `stream` current until the end of the scope, when it is not the
// current one already (a caller on a multi-GPU host may pass a stream of another device than the
// thread's current one, e.g. a layer placed on GPU 1 called while GPU 0 is current): the kernel
// then runs where the stream and its buffers are. The null stream belongs to the current device.
class StreamDeviceScope {
 public:
  explicit StreamDeviceScope(hipStream_t stream) {
    int sd = 0, cur = 0;
    if (stream == nullptr || hipStreamGetDevice(stream, &sd) != hipSuccess || hipGetDevice(&cur) != hipSuccess ||
        sd == cur)
      return;
    if (hipSetDevice(sd) == hipSuccess) prev_ = cur;
  }
  ~StreamDeviceScope() {
    if (prev_ >= 0) (void)hipSetDevice(prev_);
  }
  StreamDeviceScope(const StreamDeviceScope&) = delete;
  StreamDeviceScope& operator=(const StreamDeviceScope&) = delete;

 private:
  int prev_ = -1;
};

// Launch `kern` with hipLaunchKernel on `stream`'s device, so the launch status comes back as a
// value (a positive hipError_t), not through the sticky per-thread error state.
template <typename... KArgs>
static inline int launch(void (*kern)(KArgs...), dim3 grid, dim3 block, hipStream_t stream,
                         typename identity<KArgs>::type... args) {
  void* argv[] = {static_cast<void*>(&args)...};
  StreamDeviceScope on_stream_device(stream);
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(kern), grid, block, argv, 0, stream);
  return static_cast<int>(err);
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Per-tile arrival counters at the head of a workspace, one per 256 bytes: counters that share a
// cache line serialize their atomics in one memory-side atomic unit, and every workgroup of a
// split kernel arrives at about the same time.
constexpr int kCounterStride = 64;  // uint32 elements between consecutive counters
static inline size_t counter_bytes(size_t ntiles) { return ntiles * kCounterStride * sizeof(uint32_t); }

__host__ __device__ inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// ---- data exchanged between the workgroups of one kernel (split reductions) ----
//
// A workgroup publishes its partial sums, then bumps a per-tile arrival counter; the workgroup
// that arrives last adds everything up. The partials are written and read with device-coherent
// accesses (agent-scope atomic loads/stores for 4 bytes, buffer accesses with the sc1 cache
// policy for 16 bytes -- the same instructions), which bypass the XCD-private L2 state. Ordering
// then needs no agent-scope release/acquire fence (those write back and invalidate the whole L2
// of every XCD and cost several microseconds per workgroup): each thread waits for its own
// coherent stores to complete before the workgroup barrier, the counter increment follows the
// barrier, and the last arriver issues its coherent loads only after it has seen the final count.

__device__ inline void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kCpolSc1 = 16;                   // cache policy bits: sc1 (device coherent)
constexpr int kRawBufferDword3 = 0x00020000;   // raw (untyped) buffer descriptor word 3

// A buffer resource over [base, base + bytes) for 16-byte coherent accesses (bytes < 2^31).
__device__ inline __amdgpu_buffer_rsrc_t coherent_rsrc(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(bytes), kRawBufferDword3);
}
__device__ inline void store_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, static_cast<int>(byte_off), 0, kCpolSc1);
}
__device__ inline float4v load_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(byte_off), 0, kCpolSc1));
}

// Every thread of the workgroup calls this after its coherent stores. Returns true in every
// thread of the workgroup that arrives last for `counter` (the expected-th arrival); that
// workgroup must call reset_counter() so the counter is zero again for the next launch.
__device__ inline bool arrive_last_coherent(uint32_t* counter, uint32_t expected) {
  __shared__ uint32_t s_last;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed at the coherence point
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev + 1u == expected) ? 1u : 0u;
  }
  __syncthreads();
  return s_last != 0u;
}

__device__ inline void reset_counter(uint32_t* counter) {
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tile-packed operand layout of the 256x256 GEMM (activations from the rowscale cast, weights from
// g16_pack_weight). An operand with R rows (rows = M for activations, N for the transposed
// weight) and K columns is stored as blocks of kPackRows rows x kPackK columns; block (t, ks) is at
// block index t * ceil(K / kPackK) + ks, 16 KB each. Inside a block, 16-byte chunk q*64 + i
// (q < 16, i < 64) holds columns 8*((i % 4) ^ pack_swz(r)) .. +7 of local row r = 16q + i/4.
// Rows >= R and columns >= K are zero. This is the GEMM's LDS stage image, so its DMA copies whole
// 1 KB runs.
constexpr int kPackRows = 256, kPackK = 32;
// Chunk swizzle of that image: row r keeps its 8-column group c at chunk position c ^ pack_swz(r).
// The 256x256 GEMM reads a 16x32 MFMA operand as one 16-byte LDS read per lane (lane l: row
// 16q + l % 16, group l / 16). On gfx950 that read is conflict-free with this swizzle; with
// (r / 4) % 4, which spreads each 16 lanes over all 64 banks, the LDS serialised it 2-way
// (measured: 8.0 instead of 4.06 cycles per read instruction when the LDS is saturated).
__host__ __device__ constexpr int pack_swz(int r) { return (r >> 1) & 3; }
__host__ __device__ inline int packed_ksteps(int K) { return (K + kPackK - 1) / kPackK; }
__host__ __device__ inline size_t packed_bytes_for(int R, int K) {
  return static_cast<size_t>((R + kPackRows - 1) / kPackRows) * packed_ksteps(K) * (kPackRows * kPackK * 2);
}
// Byte offset of 16-byte chunk `oc` (columns 8*oc .. 8*oc+7) of row `row`.
__device__ inline size_t packed_offset(int row, int oc, int nks) {
  const int t = row / kPackRows, local = row % kPackRows;
  const int q = local / 16, ks = oc / 4, cc = oc % 4;
  const int i = (local % 16) * 4 + (cc ^ pack_swz(local));
  return ((static_cast<size_t>(t) * nks + ks) * 1024 + q * 64 + i) * 16;
}

__device__ inline float h2f(_Float16 h) { return static_cast<float>(h); }
__device__ inline float to_f(float x) { return x; }
__device__ inline float to_f(_Float16 x) { return static_cast<float>(x); }

}  // namespace g16
