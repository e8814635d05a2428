// common.h -- shared types and helpers of the sparse-conv HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "sam3d_spconv_amd.h"

namespace spc {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 64-bit voxel key: b:18 | x:15 | y:15 | z:15 bits (63 bits; bit 63 clear).
constexpr int kCoordBits = 15;
constexpr int32_t kCoordLimit = 1 << kCoordBits;      // x, y, z in [0, 32768)
constexpr int32_t kBatchLimit = 1 << 18;              // b in [0, 262144)
constexpr unsigned long long kEmptyKey = ~0ull;

__host__ __device__ inline unsigned long long pack_key(int32_t b, int32_t x, int32_t y,
                                                       int32_t z) {
    return ((unsigned long long)(uint32_t)b << 45) | ((unsigned long long)(uint32_t)x << 30) |
           ((unsigned long long)(uint32_t)y << 15) | (unsigned long long)(uint32_t)z;
}

__device__ inline uint32_t hash_key(unsigned long long k) {
    // 64-bit finaliser (splitmix64 constants), folded to 32 bits
    k ^= k >> 30;
    k *= 0xbf58476d1ce4e5b9ull;
    k ^= k >> 27;
    k *= 0x94d049bb133111ebull;
    k ^= k >> 31;
    return (uint32_t)k;
}

// Workgroup barrier that orders LDS traffic only.  __syncthreads() also
// fences global memory, which makes the compiler wait for every outstanding
// global load (s_waitcnt vmcnt(0)) -- including register prefetches meant to
// stay in flight across the barrier.  The kernels' barriers protect LDS
// stages only, so an LDS-scoped fence is sufficient.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt on the vector-memory counter alone (gfx9 encoding: vmcnt in bits
// [3:0] and [15:14]; expcnt [6:4] and lgkmcnt [11:8] at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// One LDS-DMA load (gfx950 buffer_load_dwordx4 ... lds): lane l's 16 bytes
// at buffer offset voff + soff go to LDS byte address lds_addr + 16 l; an
// out-of-range offset writes zeros.  Issued from inline assembly so that the
// compiler's wait-count tracking does not make every later LDS read wait
// for it; callers wait for completion themselves (dma_barrier).  M0 needs
// one wait state before the load.
// The scalar operands pass through readfirstlane so that they are in SGPRs
// at the asm (they must be wave-uniform).
__device__ __forceinline__ void lds_dma_x4(u32x4 rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
    const u32x4 rs = {(uint32_t)__builtin_amdgcn_readfirstlane(rsrc.x),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rsrc.y),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rsrc.z),
                      (uint32_t)__builtin_amdgcn_readfirstlane(rsrc.w)};
    const uint32_t m0v = (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr);
    const uint32_t so = (uint32_t)__builtin_amdgcn_readfirstlane(soff);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(m0v), "v"(voff), "s"(rs), "s"(so)
                 : "memory", "m0");
}

// Workgroup barrier for LDS filled by LDS-DMA loads: waits until at most N
// of this wave's vector-memory loads are outstanding (the DMA loads are
// older than the last N) and its LDS operations are done, then s_barrier.
// No memory fence: a release fence on LDS would also wait for the N younger
// loads, weight prefetches meant to cross the barrier.  The signal fences
// keep the compiler from moving memory accesses across it.
template <int N>
__device__ __forceinline__ void dma_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    wait_vmcnt<N>();
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// s_waitcnt vmcnt(n) for a wave-uniform run-time n in [0, MAX]: the
// immediate comes from a chain of scalar compares.
template <int N, int MAX>
__device__ __forceinline__ void wait_vmcnt_le(int n) {
    if constexpr (N >= MAX) {
        wait_vmcnt<MAX>();
    } else {
        if (n <= N) wait_vmcnt<N>();
        else wait_vmcnt_le<N + 1, MAX>(n);
    }
}

// dma_barrier for a run-time count n <= MAX of younger loads.
template <int MAX>
__device__ __forceinline__ void dma_barrier_le(int n) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    wait_vmcnt_le<0, MAX>(n);
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Round-to-nearest-even float -> bf16 / f16 bits (device): the gfx950
// hardware converts (v_cvt_pk_bf16_f32, v_cvt_f16_f32); NaNs stay NaNs.
__device__ inline uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ inline float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ inline uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}
__device__ inline float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// x * sigmoid(x) = x / (1 + e^-x) with the hardware exp2 and reciprocal
// (each within a few F32 ulps; the results are rounded to bf16 / f16 or
// compared with a tolerance).
__device__ inline float silu_f32(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves aligned sub-buffers out of a caller-owned workspace.
struct Carver {
    char* base;
    size_t cap;
    size_t used = 0;
    bool ok = true;
    Carver(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
    template <typename T>
    T* take(size_t count) {
        used = align_up(used, 256);
        T* p = reinterpret_cast<T*>(base + used);
        used += count * sizeof(T);
        if (used > cap || (base == nullptr && count > 0)) ok = false;
        return p;
    }
};

// Byte counter mirroring Carver for workspace-size queries.
struct Sizer {
    size_t used = 0;
    template <typename T>
    T* take(size_t count) {
        used = align_up(used, 256);
        used += count * sizeof(T);
        return nullptr;
    }
};

// Device status word layout (first int of every workspace).
constexpr int kStatusBytes = 256;

void set_last_error(const char* fmt, ...);
void clear_last_error();
int hip_status(hipError_t e, const char* what);

// Shared device utilities (maps.hip / sort.hip).
hipError_t fill_i32(hipStream_t s, int32_t* p, int32_t v, int64_t n);
hipError_t fill_u64(hipStream_t s, unsigned long long* p, unsigned long long v, int64_t n);
hipError_t iota_i32(hipStream_t s, int32_t* p, int64_t n);

// Stable LSD radix sort of (key, value) pairs over key bits [0, end_bit).
// vals_in may be null (values = 0..n-1).  keys_out / vals_out may alias
// nothing else.  Workspace from radix_sort_ws_bytes.
size_t radix_sort_ws_bytes(int64_t n, int key_bytes);
hipError_t radix_sort_u32(hipStream_t s, const uint32_t* keys_in, const int32_t* vals_in,
                          uint32_t* keys_out, int32_t* vals_out, int64_t n, int end_bit, void* ws,
                          size_t ws_bytes);
hipError_t radix_sort_u64(hipStream_t s, const unsigned long long* keys_in,
                          const int32_t* vals_in, unsigned long long* keys_out, int32_t* vals_out,
                          int64_t n, int end_bit, void* ws, size_t ws_bytes);

// Exclusive prefix sum of int32 (n elements) with total written to *total.
size_t scan_ws_bytes(int64_t n);
hipError_t exclusive_scan_i32(hipStream_t s, const int32_t* in, int32_t* out, int32_t* total,
                              int64_t n, void* ws, size_t ws_bytes);

}  // namespace spc

#define SPC_HIP(call)                                             \
    do {                                                          \
        hipError_t e_ = (call);                                   \
        if (e_ != hipSuccess) return spc::hip_status(e_, #call);  \
    } while (0)
