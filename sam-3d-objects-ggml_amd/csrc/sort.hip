// sort.hip -- device utilities: stable LSD radix sort of (key, value) pairs,
// exclusive scans, fills, and the library's error plumbing.
//
// The radix sort is what makes the kernel map bit-exact with the
// reference's std::stable_sort of tokens by mask (SRC/sparse_ops.cpp:143-
// 145): LSD radix sort is stable per pass, ties keep input order, and the
// input order is token order, so (mask, token) comes out exactly as
// std::stable_sort orders it.
//
// Per pass (8-bit digit, 256 bins):
//   upsweep   : per-tile digit histogram (tile = 256 threads x 8 keys)
//   scan      : one workgroup turns the digit-major [256 x tiles] counts
//               into exclusive global offsets
//   downsweep : per tile, stable rank of every key among equal digits via
//               64-lane ballots (peer mask -> popcount of lower lanes), wave
//               counts combined in LDS, scattered to offset + rank
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace spc {

namespace {

thread_local char g_last_error[512] = "";

constexpr int kRsThreads = 256;
constexpr int kRsItems = 8;
constexpr int kRsTile = kRsThreads * kRsItems;
constexpr int kRsBins = 256;
constexpr int kRsWaves = kRsThreads / 64;

template <typename K>
__global__ __launch_bounds__(kRsThreads) void rs_upsweep(const K* __restrict__ keys, int64_t n,
                                                         int shift, int32_t* __restrict__ counts,
                                                         int nblocks) {
    __shared__ int32_t hist[kRsBins];
    hist[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kRsTile;
#pragma unroll
    for (int r = 0; r < kRsItems; ++r) {
        const int64_t i = base + r * kRsThreads + threadIdx.x;
        if (i < n) {
            const uint32_t d = (uint32_t)(keys[i] >> shift) & (kRsBins - 1);
            atomicAdd(&hist[d], 1);
        }
    }
    __syncthreads();
    counts[(int64_t)threadIdx.x * nblocks + blockIdx.x] = hist[threadIdx.x];
}

template <typename K>
__global__ __launch_bounds__(kRsThreads) void rs_downsweep(
    const K* __restrict__ keys_in, const int32_t* __restrict__ vals_in, K* __restrict__ keys_out,
    int32_t* __restrict__ vals_out, int64_t n, int shift, const int32_t* __restrict__ offsets,
    int nblocks) {
    __shared__ int32_t wave_off[kRsWaves][kRsBins];
    __shared__ int32_t run[kRsBins];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    run[tid] = offsets[(int64_t)tid * nblocks + blockIdx.x];
    const int64_t base = (int64_t)blockIdx.x * kRsTile;
    const unsigned long long lower = (1ull << lane) - 1ull;
    for (int r = 0; r < kRsItems; ++r) {
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) wave_off[w][tid] = 0;
        __syncthreads();
        const int64_t i = base + r * kRsThreads + tid;
        const bool valid = i < n;
        const K key = valid ? keys_in[i] : (K)0;
        const int32_t val = valid ? (vals_in ? vals_in[i] : (int32_t)i) : 0;
        const uint32_t d = (uint32_t)(key >> shift) & (kRsBins - 1);
        // lanes of this wave holding the same digit
        unsigned long long peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const unsigned long long bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        const int rank = __popcll(peers & lower);
        if (valid && rank == 0) wave_off[wave][d] = __popcll(peers);
        __syncthreads();
        {
            // thread tid owns digit tid: wave counts -> offsets (global base +
            // keys of this digit already placed by earlier rounds)
            int32_t acc = run[tid];
#pragma unroll
            for (int w = 0; w < kRsWaves; ++w) {
                const int32_t c = wave_off[w][tid];
                wave_off[w][tid] = acc;
                acc += c;
            }
            run[tid] = acc;
        }
        __syncthreads();
        if (valid) {
            const int32_t dst = wave_off[wave][d] + rank;
            keys_out[dst] = key;
            vals_out[dst] = val;
        }
        __syncthreads();
    }
}

// Exclusive scan of L int32 with one 1024-thread workgroup (contiguous
// chunk per thread, Hillis-Steele across the chunk sums).  In-place safe.
__global__ __launch_bounds__(1024) void scan_one_block(const int32_t* in, int32_t* out,
                                                       int32_t* total, int64_t len) {
    __shared__ int32_t s[1024];
    const int tid = threadIdx.x;
    const int64_t per = (len + 1023) / 1024;
    const int64_t b = tid * per;
    const int64_t e = b + per < len ? b + per : len;
    int32_t sum = 0;
    for (int64_t i = b; i < e; ++i) sum += in[i];
    s[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int32_t v = tid >= off ? s[tid - off] : 0;
        __syncthreads();
        s[tid] += v;
        __syncthreads();
    }
    int32_t acc = s[tid] - sum;
    for (int64_t i = b; i < e; ++i) {
        const int32_t v = in[i];
        out[i] = acc;
        acc += v;
    }
    if (tid == 1023 && total) *total = s[1023];
}

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

__global__ __launch_bounds__(kScanThreads) void scan_tile_sums(const int32_t* __restrict__ in,
                                                               int32_t* __restrict__ sums,
                                                               int64_t n) {
    __shared__ int32_t s[kScanThreads];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int32_t acc = 0;
    for (int r = 0; r < kScanItems; ++r) {
        const int64_t i = base + r * kScanThreads + threadIdx.x;
        if (i < n) acc += in[i];
    }
    s[threadIdx.x] = acc;
    __syncthreads();
    for (int w = kScanThreads / 2; w > 0; w >>= 1) {
        if (threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) sums[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(kScanThreads) void scan_tiles(const int32_t* __restrict__ in,
                                                           int32_t* __restrict__ out,
                                                           const int32_t* __restrict__ tile_off,
                                                           int64_t n) {
    __shared__ int32_t s[kScanThreads];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int32_t v[kScanItems];
    int32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        v[j] = i < n ? in[i] : 0;
        sum += v[j];
    }
    s[threadIdx.x] = sum;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {
        const int32_t t = threadIdx.x >= off ? s[threadIdx.x - off] : 0;
        __syncthreads();
        s[threadIdx.x] += t;
        __syncthreads();
    }
    int32_t acc = tile_off[blockIdx.x] + s[threadIdx.x] - sum;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        if (i < n) out[i] = acc;
        acc += v[j];
    }
}

template <typename T>
__global__ void fill_kernel(T* p, T v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void iota_kernel(int32_t* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (int32_t)i;
}

inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

template <typename K>
hipError_t radix_sort(hipStream_t s, const K* keys_in, const int32_t* vals_in, K* keys_out,
                      int32_t* vals_out, int64_t n, int end_bit, void* ws, size_t ws_bytes) {
    if (n <= 0) return hipSuccess;
    const int nblocks = (int)ceil_div(n, kRsTile);
    Carver c(ws, ws_bytes);
    int32_t* counts = c.take<int32_t>((size_t)kRsBins * nblocks);
    K* tk[2] = {c.take<K>(n), c.take<K>(n)};
    int32_t* tv[2] = {c.take<int32_t>(n), c.take<int32_t>(n)};
    if (!c.ok) return hipErrorInvalidValue;
    int passes = (end_bit + 7) / 8;
    if (passes < 1) passes = 1;
    const K* kin = keys_in;
    const int32_t* vin = vals_in;
    for (int p = 0; p < passes; ++p) {
        const bool last = p == passes - 1;
        K* kout = last ? keys_out : tk[p & 1];
        int32_t* vout = last ? vals_out : tv[p & 1];
        const int shift = p * 8;
        rs_upsweep<K><<<nblocks, kRsThreads, 0, s>>>(kin, n, shift, counts, nblocks);
        scan_one_block<<<1, 1024, 0, s>>>(counts, counts, nullptr, (int64_t)kRsBins * nblocks);
        rs_downsweep<K><<<nblocks, kRsThreads, 0, s>>>(kin, vin, kout, vout, n, shift, counts,
                                                       nblocks);
        kin = kout;
        vin = vout;
    }
    return hipGetLastError();
}

}  // namespace

void set_last_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
    set_last_error("%s failed: %s", what, hipGetErrorString(e));
    return SPC_HIP_ERROR;
}

hipError_t fill_i32(hipStream_t s, int32_t* p, int32_t v, int64_t n) {
    if (n <= 0) return hipSuccess;
    fill_kernel<int32_t><<<grid_for(n, 256), 256, 0, s>>>(p, v, n);
    return hipGetLastError();
}

hipError_t fill_u64(hipStream_t s, unsigned long long* p, unsigned long long v, int64_t n) {
    if (n <= 0) return hipSuccess;
    fill_kernel<unsigned long long><<<grid_for(n, 256), 256, 0, s>>>(p, v, n);
    return hipGetLastError();
}

hipError_t iota_i32(hipStream_t s, int32_t* p, int64_t n) {
    if (n <= 0) return hipSuccess;
    iota_kernel<<<grid_for(n, 256), 256, 0, s>>>(p, n);
    return hipGetLastError();
}

size_t radix_sort_ws_bytes(int64_t n, int key_bytes) {
    const int64_t nblocks = ceil_div(n > 0 ? n : 1, kRsTile);
    Sizer z;
    z.take<int32_t>((size_t)kRsBins * nblocks);
    for (int i = 0; i < 2; ++i) z.take<char>((size_t)n * key_bytes);
    for (int i = 0; i < 2; ++i) z.take<int32_t>(n);
    return z.used + 256;
}

hipError_t radix_sort_u32(hipStream_t s, const uint32_t* keys_in, const int32_t* vals_in,
                          uint32_t* keys_out, int32_t* vals_out, int64_t n, int end_bit, void* ws,
                          size_t ws_bytes) {
    return radix_sort<uint32_t>(s, keys_in, vals_in, keys_out, vals_out, n, end_bit, ws, ws_bytes);
}

hipError_t radix_sort_u64(hipStream_t s, const unsigned long long* keys_in,
                          const int32_t* vals_in, unsigned long long* keys_out, int32_t* vals_out,
                          int64_t n, int end_bit, void* ws, size_t ws_bytes) {
    return radix_sort<unsigned long long>(s, keys_in, vals_in, keys_out, vals_out, n, end_bit, ws,
                                          ws_bytes);
}

size_t scan_ws_bytes(int64_t n) {
    Sizer z;
    z.take<int32_t>(ceil_div(n > 0 ? n : 1, kScanTile) + 1);
    return z.used + 256;
}

hipError_t exclusive_scan_i32(hipStream_t s, const int32_t* in, int32_t* out, int32_t* total,
                              int64_t n, void* ws, size_t ws_bytes) {
    if (n <= 0) return total ? fill_i32(s, total, 0, 1) : hipSuccess;
    if (n <= 65536) {
        scan_one_block<<<1, 1024, 0, s>>>(in, out, total, n);
        return hipGetLastError();
    }
    const int64_t tiles = ceil_div(n, kScanTile);
    Carver c(ws, ws_bytes);
    int32_t* sums = c.take<int32_t>(tiles + 1);
    if (!c.ok) return hipErrorInvalidValue;
    scan_tile_sums<<<(unsigned)tiles, kScanThreads, 0, s>>>(in, sums, n);
    scan_one_block<<<1, 1024, 0, s>>>(sums, sums, total, tiles);
    scan_tiles<<<(unsigned)tiles, kScanThreads, 0, s>>>(in, out, sums, n);
    return hipGetLastError();
}

}  // namespace spc

extern "C" {

const char* spc_last_error(void) { return spc::g_last_error; }

const char* spc_status_string(int status) {
    switch (status) {
        case SPC_OK: return "ok";
        case SPC_BAD_SHAPE: return "bad shape";
        case SPC_BAD_COORD: return "coordinate out of range";
        case SPC_DUP_COORD: return "duplicate coordinate";
        case SPC_OOM: return "workspace too small";
        case SPC_HIP_ERROR: return "HIP error";
        case SPC_BAD_ARG: return "bad argument";
        default: return "unknown status";
    }
}

int spc_version(void) { return 1; }

}  // extern "C"
