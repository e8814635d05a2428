// sort.hip -- device utilities: stable LSD radix sort of (key, value) pairs,
// exclusive scans, fills, and the library's error plumbing.
//
// The radix sort is what makes the kernel map bit-exact with the
// reference's std::stable_sort of tokens by mask (SRC/sparse_ops.cpp:143-
// 145): LSD radix sort is stable per pass, ties keep input order, and the
// input order is token order, so (mask, token) comes out exactly as
// std::stable_sort orders it.
//
// Per pass (9-bit digit, 512 bins; 27-bit masks take 3 passes):
//   upsweep   : per-tile digit histogram (tile = 256 threads x 1-8 keys:
//               small sorts take fewer keys per thread, up to 64 tiles)
//   offsets   : up to 128 tiles, every downsweep block derives its own
//               offsets from the block-major [tiles x 512] counts (a wave
//               reads 512 contiguous bytes per tile, up to 64 tiles in one
//               batch of loads); beyond that the counts are digit-major and
//               a multi-block exclusive scan turns them into offsets
//   downsweep : per tile, stable rank of every key among equal digits via
//               64-lane ballots (peer mask -> popcount of lower lanes); the
//               per-(round, wave) digit counts of up to four rounds are
//               scanned in one LDS pass (three barriers per 1,024 keys);
//               scattered to offset + rank
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace spc {

namespace {

thread_local char g_last_error[512] = "";

constexpr int kRsThreads = 256;
constexpr int kRsItems = 8;                 // keys per thread of large sorts
constexpr int kRsBits = 9;                 // digit bits: 27-bit masks sort in 3 passes
constexpr int kRsBins = 1 << kRsBits;
constexpr int kRsWaves = kRsThreads / 64;
constexpr int kRsBinsPerThread = kRsBins / kRsThreads;
constexpr int kRsFusedBlocks = 128;        // up to here each downsweep block scans the counts
constexpr int kRsSpreadBlocks = 64;        // small sorts: fewer keys per thread up to this many tiles

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ inline int32_t wave_incl_scan(int32_t v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int32_t t = __shfl_up(v, off);
        if (lane >= off) v += t;
    }
    return v;
}

// Per-tile digit histogram, digit-major (counts[d * nblocks + block], the
// order a global scan needs) or, with BLOCK_MAJOR, one row of kRsBins per
// tile (counts[block * kRsBins + d]: the fused downsweep's coalesced reads).
// A tile is kRsThreads x ITEMS keys.
template <typename K, int ITEMS, bool BLOCK_MAJOR>
__global__ __launch_bounds__(kRsThreads) void rs_upsweep(const K* __restrict__ keys, int64_t n,
                                                         int shift, int32_t* __restrict__ counts,
                                                         int nblocks) {
    __shared__ int32_t hist[kRsBins];
#pragma unroll
    for (int j = 0; j < kRsBinsPerThread; ++j) hist[j * kRsThreads + threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * (kRsThreads * ITEMS);
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const int64_t i = base + r * kRsThreads + threadIdx.x;
        if (i < n) {
            const uint32_t d = (uint32_t)(keys[i] >> shift) & (kRsBins - 1);
            atomicAdd(&hist[d], 1);
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRsBinsPerThread; ++j) {
        const int d = j * kRsThreads + threadIdx.x;
        counts[BLOCK_MAJOR ? (int64_t)blockIdx.x * kRsBins + d : (int64_t)d * nblocks + blockIdx.x] =
            hist[d];
    }
}

// Stable scatter of one tile.  `offsets` (digit-major, as the scan leaves
// them) gives each (digit, block) its first output position; with
// FUSED the block derives its own offsets from the raw block-major counts
// instead: offset(d) = (keys of smaller digits) + (keys of digit d in
// earlier blocks).  Within the tile every key is ranked among equal digits by
// 64-lane ballots (peer mask -> popcount of lower lanes); the counts of
// each (round, wave) become offsets in input order (round, then wave), up
// to four rounds per group.
template <typename K, bool FUSED, int ITEMS>
__global__ __launch_bounds__(kRsThreads) void rs_downsweep(
    const K* __restrict__ keys_in, const int32_t* __restrict__ vals_in, K* __restrict__ keys_out,
    int32_t* __restrict__ vals_out, int64_t n, int shift, const int32_t* __restrict__ offsets,
    int nblocks) {
    constexpr int R = ITEMS < 4 ? ITEMS : 4;  // rounds per group
    __shared__ int32_t cnt[R * kRsWaves][kRsBins];
    __shared__ int32_t run[kRsBins];
    __shared__ int32_t wsum[kRsWaves];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t base = (int64_t)blockIdx.x * (kRsThreads * ITEMS);
    // FUSED: thread tid owns digits 2 tid and 2 tid + 1, one 8-byte load per
    // block's row of counts (a wave's load is 512 contiguous bytes).  Up to
    // 64 loads go out at once (one batch up to 64 blocks), the row index
    // clamped so every load is in bounds; the first batch before the tile's
    // keys, so both latencies overlap.
    static_assert(kRsBinsPerThread == 2, "two digits per thread");
    constexpr int MAXB = 64;
    const int2* c = reinterpret_cast<const int2*>(offsets) + tid;
    int2 v2[FUSED ? MAXB : 1];
    if constexpr (FUSED) {
#pragma unroll
        for (int k = 0; k < MAXB; ++k) v2[k] = c[(int64_t)min(k, nblocks - 1) * (kRsBins / 2)];
    }
    K key[ITEMS];
    int32_t val[ITEMS];
#pragma unroll
    for (int r = 0; r < ITEMS; ++r) {
        const int64_t i = base + r * kRsThreads + tid;
        const bool valid = i < n;
        key[r] = valid ? keys_in[i] : (K)0;
        val[r] = valid ? (vals_in ? vals_in[i] : (int32_t)i) : 0;
    }
    if constexpr (FUSED) {
        int32_t tot[2] = {0, 0}, before[2] = {0, 0};
        for (int b0 = 0;;) {
#pragma unroll
            for (int k = 0; k < MAXB; ++k) {
                const int b = b0 + k;
                if (b < nblocks) {
                    tot[0] += v2[k].x;
                    tot[1] += v2[k].y;
                    if (b < (int)blockIdx.x) {
                        before[0] += v2[k].x;
                        before[1] += v2[k].y;
                    }
                }
            }
            b0 += MAXB;
            if (b0 >= nblocks) break;
#pragma unroll
            for (int k = 0; k < MAXB; ++k)
                v2[k] = c[(int64_t)min(b0 + k, nblocks - 1) * (kRsBins / 2)];
        }
        const int32_t mine = tot[0] + tot[1];
        const int32_t incl = wave_incl_scan(mine, lane);
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int32_t excl = incl - mine;
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w)
            if (w < wave) excl += wsum[w];
        run[2 * tid] = excl + before[0];
        run[2 * tid + 1] = excl + tot[0] + before[1];
    } else {
#pragma unroll
        for (int j = 0; j < kRsBinsPerThread; ++j) {
            const int d = j * kRsThreads + tid;
            run[d] = offsets[(int64_t)d * nblocks + blockIdx.x];
        }
    }
    const unsigned long long lower = (1ull << lane) - 1ull;
#pragma unroll
    for (int g = 0; g < ITEMS / R; ++g) {
#pragma unroll
        for (int e = 0; e < R * kRsWaves; ++e)
#pragma unroll
            for (int j = 0; j < kRsBinsPerThread; ++j) cnt[e][j * kRsThreads + tid] = 0;
        __syncthreads();  // also orders run[] (written per owner above) before the scan
        uint32_t dig[R];
        int rank[R];
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const int r = g * R + q;
            const bool valid = base + r * kRsThreads + tid < n;
            dig[q] = (uint32_t)(key[r] >> shift) & (kRsBins - 1);
            // lanes of this wave holding the same digit
            unsigned long long peers = __ballot(valid);
#pragma unroll
            for (int b = 0; b < kRsBits; ++b) {
                const bool bit = (dig[q] >> b) & 1u;
                const unsigned long long bal = __ballot(bit);
                peers &= bit ? bal : ~bal;
            }
            rank[q] = __popcll(peers & lower);
            if (valid && rank[q] == 0) cnt[q * kRsWaves + wave][dig[q]] = __popcll(peers);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kRsBinsPerThread; ++j) {
            // (round, wave) counts -> offsets in input order, after the keys
            // of this digit placed by earlier groups
            const int dd = j * kRsThreads + tid;
            int32_t acc = run[dd];
#pragma unroll
            for (int e = 0; e < R * kRsWaves; ++e) {
                const int32_t c = cnt[e][dd];
                cnt[e][dd] = acc;
                acc += c;
            }
            run[dd] = acc;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const int r = g * R + q;
            if (base + r * kRsThreads + tid < n) {
                const int32_t dst = cnt[q * kRsWaves + wave][dig[q]] + rank[q];
                keys_out[dst] = key[r];
                vals_out[dst] = val[r];
            }
        }
        if (g + 1 < ITEMS / R) __syncthreads();  // cnt is cleared by the next group
    }
}

// Exclusive scan of len int32 with one 1024-thread workgroup: rounds of
// 4096 elements (4 contiguous per thread), wave shuffles and one LDS step per
// round, a running carry across rounds.  In-place safe.
__global__ __launch_bounds__(1024) void scan_one_block(const int32_t* in, int32_t* out,
                                                       int32_t* total, int64_t len) {
    constexpr int IT = 4;
    __shared__ int32_t wsum[16];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int32_t carry = 0;
    for (int64_t base = 0; base < len; base += 1024 * IT) {
        int32_t v[IT];
        int32_t mine = 0;
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int64_t i = base + (int64_t)tid * IT + j;
            v[j] = i < len ? in[i] : 0;
            mine += v[j];
        }
        const int32_t incl = wave_incl_scan(mine, lane);
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int32_t excl = carry + incl - mine;
        int32_t round_total = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            if (w < wave) excl += wsum[w];
            round_total += wsum[w];
        }
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const int64_t i = base + (int64_t)tid * IT + j;
            if (i < len) out[i] = excl;
            excl += v[j];
        }
        carry += round_total;
        __syncthreads();  // wsum is rewritten by the next round
    }
    if (tid == 0 && total) *total = carry;
}

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

// Sum of each tile of kScanTile values: per-thread sums, wave shuffles,
// one LDS step.
__global__ __launch_bounds__(kScanThreads) void scan_tile_sums(const int32_t* __restrict__ in,
                                                               int32_t* __restrict__ sums,
                                                               int64_t n) {
    __shared__ int32_t wsum[kScanThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int32_t acc = 0;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        const int64_t i = base + r * kScanThreads + threadIdx.x;
        if (i < n) acc += in[i];
    }
    const int32_t incl = wave_incl_scan(acc, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t t = 0;
#pragma unroll
        for (int w = 0; w < kScanThreads / 64; ++w) t += wsum[w];
        sums[blockIdx.x] = t;
    }
}

// Exclusive scan of each tile (kScanItems contiguous values per thread)
// from its offset tile_off[tile]: wave shuffles and one LDS step.
__global__ __launch_bounds__(kScanThreads) void scan_tiles(const int32_t* __restrict__ in,
                                                           int32_t* __restrict__ out,
                                                           const int32_t* __restrict__ tile_off,
                                                           int64_t n) {
    __shared__ int32_t wsum[kScanThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int32_t v[kScanItems];
    int32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        v[j] = i < n ? in[i] : 0;
        sum += v[j];
    }
    const int32_t incl = wave_incl_scan(sum, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int32_t acc = tile_off[blockIdx.x] + incl - sum;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w)
        if (w < wave) acc += wsum[w];
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

// Keys per thread: the fewest that keep at most kRsSpreadBlocks tiles (small
// sorts spread over more compute units); large sorts take kRsItems.
inline int rs_items(int64_t n) {
    for (int it = 1; it < kRsItems; it *= 2)
        if (ceil_div(n, (int64_t)kRsThreads * it) <= kRsSpreadBlocks) return it;
    return kRsItems;
}

template <typename K, int ITEMS>
hipError_t radix_sort_items(hipStream_t s, const K* keys_in, const int32_t* vals_in, K* keys_out,
                            int32_t* vals_out, int64_t n, int end_bit, void* ws, size_t ws_bytes) {
    const int nblocks = (int)ceil_div(n, (int64_t)kRsThreads * ITEMS);
    const bool fused = nblocks <= kRsFusedBlocks;
    Carver c(ws, ws_bytes);
    int32_t* counts = c.take<int32_t>((size_t)kRsBins * nblocks);
    K* tk[2] = {c.take<K>(n), c.take<K>(n)};
    int32_t* tv[2] = {c.take<int32_t>(n), c.take<int32_t>(n)};
    const size_t scan_bytes = fused ? 0 : scan_ws_bytes((int64_t)kRsBins * nblocks);
    char* scan_ws = c.take<char>(scan_bytes);
    if (!c.ok) return hipErrorInvalidValue;
    int passes = (end_bit + kRsBits - 1) / kRsBits;
    if (passes < 1) passes = 1;
    const K* kin = keys_in;
    const int32_t* vin = vals_in;
    for (int p = 0; p < passes; ++p) {
        const bool last = p == passes - 1;
        K* kout = last ? keys_out : tk[p & 1];
        int32_t* vout = last ? vals_out : tv[p & 1];
        const int shift = p * kRsBits;
        if (fused) {
            rs_upsweep<K, ITEMS, true><<<nblocks, kRsThreads, 0, s>>>(kin, n, shift, counts, nblocks);
            rs_downsweep<K, true, ITEMS><<<nblocks, kRsThreads, 0, s>>>(
                kin, vin, kout, vout, n, shift, counts, nblocks);
        } else {
            rs_upsweep<K, ITEMS, false><<<nblocks, kRsThreads, 0, s>>>(kin, n, shift, counts, nblocks);
            const hipError_t e = exclusive_scan_i32(s, counts, counts, nullptr,
                                                    (int64_t)kRsBins * nblocks, scan_ws, scan_bytes);
            if (e != hipSuccess) return e;
            rs_downsweep<K, false, ITEMS><<<nblocks, kRsThreads, 0, s>>>(
                kin, vin, kout, vout, n, shift, counts, nblocks);
        }
        kin = kout;
        vin = vout;
    }
    return hipGetLastError();
}

template <typename K>
hipError_t radix_sort(hipStream_t s, const K* keys_in, const int32_t* vals_in, K* keys_out,
                      int32_t* vals_out, int64_t n, int end_bit, void* ws, size_t ws_bytes) {
    if (n <= 0) return hipSuccess;
    switch (rs_items(n)) {
        case 1: return radix_sort_items<K, 1>(s, keys_in, vals_in, keys_out, vals_out, n, end_bit, ws, ws_bytes);
        case 2: return radix_sort_items<K, 2>(s, keys_in, vals_in, keys_out, vals_out, n, end_bit, ws, ws_bytes);
        case 4: return radix_sort_items<K, 4>(s, keys_in, vals_in, keys_out, vals_out, n, end_bit, ws, ws_bytes);
        default: return radix_sort_items<K, kRsItems>(s, keys_in, vals_in, keys_out, vals_out, n, end_bit, ws, ws_bytes);
    }
}

}  // namespace

void set_last_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_last_error() { g_last_error[0] = '\0'; }

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
    const int64_t m = n > 0 ? n : 1;
    const int64_t nblocks = ceil_div(m, (int64_t)kRsThreads * rs_items(m));
    Sizer z;
    z.take<int32_t>((size_t)kRsBins * nblocks);
    for (int i = 0; i < 2; ++i) z.take<char>((size_t)n * key_bytes);
    for (int i = 0; i < 2; ++i) z.take<int32_t>(n);
    z.take<char>(nblocks <= kRsFusedBlocks ? 0 : scan_ws_bytes((int64_t)kRsBins * nblocks));
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

// Up to here one workgroup scans alone (four rounds of 4,096); beyond, the
// three-launch tile scan is faster, each of the one workgroup's rounds
// costing a global-memory round trip (62,710 values: 26 us alone).
constexpr int64_t kScanOneBlockMax = 16384;

hipError_t exclusive_scan_i32(hipStream_t s, const int32_t* in, int32_t* out, int32_t* total,
                              int64_t n, void* ws, size_t ws_bytes) {
    if (n <= 0) return total ? fill_i32(s, total, 0, 1) : hipSuccess;
    if (n <= kScanOneBlockMax) {
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
