// conv.hip -- C ABI of the sparse convolution (kernel in conv_kernel.h):
// argument checks, dispatch by dtype, the MFMA-fragment weight packer, the
// Q8_0 block repacker and the reference-compatible spconv bridge.
#include <atomic>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "conv_kernel.h"

namespace spc {

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Clears the marker of `tiles` plan tiles (a section its builder skipped):
// convs over them set their tiles up themselves.
__global__ void plan_unmark_kernel(char* plan, int64_t tiles, int64_t tile_bytes) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < tiles) reinterpret_cast<int32_t*>(plan + t * tile_bytes)[3] = 0;
}

template <typename T, bool Q8>
size_t packed_quant_bytes(int64_t ntaps, int64_t cin, int64_t cout) {
    return (size_t)ntaps * cin * cout * Panel<T, Q8>::WB;
}

// Element strides of a stored weight tensor per layout (SPC_W_KRSC / TCK / TKC).
struct WStride {
    int64_t co, o, ci;
};
__host__ __device__ WStride weight_strides(int layout, int64_t ntaps, int64_t cin, int64_t cout) {
    if (layout == SPC_W_TCK) return {cin, cout * cin, 1};
    if (layout == SPC_W_TKC) return {1, cin * cout, cout};
    return {ntaps * cin, cin, 1};  // SPC_W_KRSC
}

// Panel word `id` (panel (tap, chunk, c32), word g, lane) of the packed
// weights: fragments g G .. g G + G - 1, each EPL elements of one output
// channel (Panel::co_of / ci_of).
template <typename T, bool Q8>
__device__ __forceinline__ void pack_word(const uint8_t* __restrict__ w, u32x4* __restrict__ out,
                                          int ntaps, int cin, int cout, WStride st, int64_t id) {
    using P = Panel<T, Q8>;
    const int kch = cin / P::KC;
    const int ncol32 = cout / 32;
    const int64_t words = (int64_t)ntaps * kch * ncol32 * P::NG * 64;
    if (id >= words) return;
    const int lane = (int)(id % 64);
    const int64_t rest = id / 64;
    const int g = (int)(rest % P::NG);
    const int64_t panel = rest / P::NG;
    const int c32 = (int)(panel % ncol32);
    const int64_t tk = panel / ncol32;
    const int kc = (int)(tk % kch);
    const int o = (int)(tk / kch);
    if constexpr (!Q8 && sizeof(T) == 2) {
        if (st.ci == 1 && ((uintptr_t)w & 15u) == 0) {
            // the word's 8 channels are contiguous: one 16-byte load
            // (16-byte aligned: cin and the chunk offsets are multiples of 8)
            const int64_t co = c32 * 32 + P::co_of(g, lane);
            const int64_t el = co * st.co + o * st.o + (int64_t)kc * P::KC + P::ci_of(g, lane);
            out[id] = *reinterpret_cast<const u32x4*>(w + el * 2);
            return;
        }
    }
    uint8_t bytes[16];
#pragma unroll
    for (int i = 0; i < P::G; ++i) {
        const int f = g * P::G + i;
        const int64_t co = c32 * 32 + P::co_of(f, lane);
        const int64_t ci0 = (int64_t)kc * P::KC + P::ci_of(f, lane);
#pragma unroll
        for (int e = 0; e < P::EPL; ++e) {
            const int64_t el = co * st.co + o * st.o + (ci0 + e) * st.ci;
#pragma unroll
            for (int b = 0; b < P::WB; ++b)
                bytes[(i * P::EPL + e) * P::WB + b] = w[el * P::WB + b];
        }
    }
    uint32_t v[4];
#pragma unroll
    for (int h = 0; h < 4; ++h)
        v[h] = (uint32_t)bytes[4 * h] | ((uint32_t)bytes[4 * h + 1] << 8) |
               ((uint32_t)bytes[4 * h + 2] << 16) | ((uint32_t)bytes[4 * h + 3] << 24);
    out[id] = u32x4{v[0], v[1], v[2], v[3]};
}

// One thread per 16-byte panel word.
template <typename T, bool Q8>
__global__ void pack_weights_kernel(const uint8_t* __restrict__ w, u32x4* __restrict__ out,
                                    int ntaps, int cin, int cout, WStride st) {
    pack_word<T, Q8>(w, out, ntaps, cin, cout, st, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

// Q8_0 scales as f32 per (tap, chunk, co): a 32-channel chunk is one block
// (block index = element index of its first channel / 32; channels run
// contiguously, st.ci == 1).
__global__ void pack_scales_kernel(const uint16_t* __restrict__ d, float* __restrict__ out,
                                   int ntaps, int cin, int cout, WStride st) {
    const int kch = cin / 32;
    const int64_t n = (int64_t)ntaps * kch * cout;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n) return;
    const int co = (int)(id % cout);
    const int64_t tk = id / cout;
    const int kc = (int)(tk % kch);
    const int o = (int)(tk / kch);
    out[id] = f16_bits_to_f32(d[(co * st.co + o * st.o + (int64_t)kc * 32) >> 5]);
}

// Packed Q8_0 panels -> packed bf16 panels of the same (tap, chunk, c32)
// order.  A Q8_0 panel holds one 16-byte word per lane (the 8 quants of
// both 16-channel blocks), a bf16 panel two (one per block); lane l's
// quants in block h belong to output channel 32 c32 + 16 h + l % 16, whose
// f32 scale they take.  One thread per panel lane: 16 quant bytes and two
// scales in, 32 bytes out, all coalesced.
// F16: the same panels of f16(f32(d) * q) (bf16 and f16 panels share the
// packed layout).
template <bool F16>
__global__ void expand_q8_0_kernel(const u32x4* __restrict__ q, const float* __restrict__ sc,
                                   u32x4* __restrict__ out, int64_t panels, int ncol32,
                                   int cout) {
    using PQ = Panel<__bf16, true>;
    using PB = Panel<__bf16, false>;
    static_assert(PQ::NG == 1 && PQ::G == 2 && PB::NG == 2 && PB::NH == 2, "Q8_0 and 16-bit panel words");
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= panels * 64) return;
    const int lane = (int)(id & 63);
    const int64_t p = id >> 6;
    const int64_t tk = p / ncol32;  // tap * chunks + chunk
    const int c32 = (int)(p - tk * ncol32);
    const float d0 = sc[tk * cout + c32 * 32 + PQ::co_of(0, lane)];
    const float d1 = sc[tk * cout + c32 * 32 + PQ::co_of(1, lane)];
    const u32x4 w = q[id];
    if constexpr (F16) {
        out[p * 128 + lane] = __builtin_bit_cast(u32x4, q8_dequant8_f16(w.x, w.y, d0));
        out[p * 128 + 64 + lane] = __builtin_bit_cast(u32x4, q8_dequant8_f16(w.z, w.w, d1));
    } else {
        out[p * 128 + lane] = __builtin_bit_cast(u32x4, q8_dequant8(w.x, w.y, d0));
        out[p * 128 + 64 + lane] = __builtin_bit_cast(u32x4, q8_dequant8(w.z, w.w, d1));
    }
}

// Element conversion between f32 / f16 / bf16 (round to nearest even), four
// elements per thread.
__device__ __forceinline__ float load_elem(const void* p, int dt, int64_t i) {
    if (dt == SPC_F32) return static_cast<const float*>(p)[i];
    const uint16_t b = static_cast<const uint16_t*>(p)[i];
    return dt == SPC_F16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b);
}
__global__ void convert_kernel(const void* __restrict__ src, int sdt, void* __restrict__ dst,
                               int ddt, int64_t n) {
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = i0 + k;
        if (i >= n) return;
        const float v = load_elem(src, sdt, i);
        if (ddt == SPC_F32) static_cast<float*>(dst)[i] = v;
        else if (ddt == SPC_F16) static_cast<uint16_t*>(dst)[i] = f32_to_f16_bits(v);
        else static_cast<uint16_t*>(dst)[i] = f32_to_bf16_bits(v);
    }
}

__global__ void q8_0_repack_kernel(const uint8_t* __restrict__ blocks, int64_t nblocks,
                                   int8_t* __restrict__ qs, uint16_t* __restrict__ d) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* src = blocks + b * 34;
    d[b] = (uint16_t)src[0] | ((uint16_t)src[1] << 8);
    uint32_t words[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        words[j] = (uint32_t)src[2 + 4 * j] | ((uint32_t)src[3 + 4 * j] << 8) |
                   ((uint32_t)src[4 + 4 * j] << 16) | ((uint32_t)src[5 + 4 * j] << 24);
    u32x4* dst = reinterpret_cast<u32x4*>(qs + b * 32);
    dst[0] = u32x4{words[0], words[1], words[2], words[3]};
    dst[1] = u32x4{words[4], words[5], words[6], words[7]};
}

// quantize_q8_0 (cpp_ggml/scripts/gguf_schema.py:14-24): one thread per
// 32-float block.  amax / 127 is an F32 division rounded to fp16; the quants
// are rint (half to even) of the F32 quotient w / f32(d), clipped to +-127.
__global__ void q8_0_quantize_kernel(const float* __restrict__ w, int64_t nblocks,
                                     uint8_t* __restrict__ blocks) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const floatx4* src = reinterpret_cast<const floatx4*>(w + b * 32);
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const floatx4 q = src[j];
        v[4 * j] = q.x;
        v[4 * j + 1] = q.y;
        v[4 * j + 2] = q.z;
        v[4 * j + 3] = q.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    if (amax == 0.0f) amax = 1e-12f;
    const uint16_t dh = f32_to_f16_bits(amax / 127.0f);
    const float d = f16_bits_to_f32(dh);
    uint8_t* dst = blocks + b * 34;
    dst[0] = (uint8_t)(dh & 0xff);
    dst[1] = (uint8_t)(dh >> 8);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        float q;
        if (d == 0.0f) {
            // amax / 127 below half the smallest fp16 subnormal rounds d to
            // 0 (always for an all-zero block): the converter's quotient is
            // +-inf, clipped to +-127, or 0/0, which its int8 cast makes 0
            q = v[j] > 0.0f ? 127.0f : (v[j] < 0.0f ? -127.0f : 0.0f);
        } else {
            q = __builtin_rintf(v[j] / d);
            q = fminf(fmaxf(q, -127.0f), 127.0f);
        }
        dst[2 + j] = (uint8_t)(int8_t)q;
    }
}

// ggml Q8_0 blocks -> f32(d) * q (exact in F32), stored as out_dtype.
__global__ void q8_0_dequant_kernel(const uint8_t* __restrict__ blocks, int64_t n,
                                    int out_dtype, void* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint8_t* blk = blocks + (i >> 5) * 34;
    const float d = f16_bits_to_f32((uint16_t)blk[0] | ((uint16_t)blk[1] << 8));
    const float v = d * (float)(int8_t)blk[2 + (i & 31)];
    if (out_dtype == SPC_F32) static_cast<float*>(out)[i] = v;
    else if (out_dtype == SPC_F16) static_cast<uint16_t*>(out)[i] = f32_to_f16_bits(v);
    else static_cast<uint16_t*>(out)[i] = f32_to_bf16_bits(v);
}

// Compute units of the current device, queried once per device (an
// unreadable attribute counts as 256, the MI355X figure).
int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// The spconv bridge's device state, one per device, grown with hipMalloc
// when a call needs more and held until the process ends (the bridge's
// signature has no workspace):
//   pack    the KRSC f16 weights packed into MFMA fragment order (every call)
//   pad     channels that are multiples of 8 but not of 32: zero-padded
//           copies of input, bias and output (widths rounded up to 32)
//   plans   self-refreshing tile plans, four entries keyed by (tokens, tile
//           geometry), least recently used replaced: a plan buffer for n
//           tokens, a copy of the index table its tiles were built from and
//           one flag per (128 rows, tap).  Each call first flags the rows
//           whose entries differ from the copy (bridge_prep_kernel); the conv
//           runs flagged tiles unplanned and writes their plan tiles and
//           entries back, so repeated calls over one index table (every conv
//           of a coordinate set) skip the tile setup, and calls that
//           alternate between token counts (the fine and coarse levels of
//           the SLAT IO blocks) keep one plan per level.
// Bridge calls on one device share it, so calls on different streams of
// one device must not overlap (one stream, as the reference's bridge
// assumes).
struct BridgePlan {
    int32_t* idx = nullptr;
    int32_t* dirty = nullptr;
    void* plan = nullptr;
    size_t idx_cap = 0;
    size_t plan_cap = 0;
    int64_t n = -1;
    int geometry = -1;  // the tile geometry whose plan section the entries describe
    uint64_t used = 0;  // last use (LRU clock)
};
constexpr int kBridgePlans = 4;
struct BridgeDev {
    void* pack = nullptr;
    size_t pack_cap = 0;
    void* pad = nullptr;
    size_t pad_cap = 0;
    BridgePlan plans[kBridgePlans];
    uint64_t clock = 0;
};

std::mutex g_bridge_mu;
BridgeDev g_bridge[64];

// Grows a held device buffer to `need` bytes (the old contents are not
// kept); false when the allocation fails.
bool bridge_grow(void*& p, size_t& cap, size_t need) {
    if (cap >= need) return true;
    // hipFree waits for the work that may still read the old buffer
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    if (hipMalloc(&p, need) != hipSuccess) {
        p = nullptr;
        (void)hipGetLastError();
        return false;
    }
    cap = need;
    return true;
}

// The bridge's per-call preparation in one launch: blocks [0, npack) pack
// the KRSC f16 weights (one thread per panel word, zeros for the padded
// channels: input channels >= cin_real or output channels >= cout_real),
// the rest flag changed index entries: dirty[27 f + o] = whether any
// offset-major entry (o, r) of [27, n] with r in [128 f, 128 f + 128)
// differs from the cached copy.  A flag block covers 256 rows, each thread
// one row across the 27 taps (all 54 loads in flight at once).
__global__ __launch_bounds__(256) void bridge_prep_kernel(
    const uint8_t* __restrict__ w, u32x4* __restrict__ packed, int cin, int cout, int cin_real,
    int cout_real, int64_t npack, const int32_t* __restrict__ idx,
    const int32_t* __restrict__ cache, int64_t n, int32_t* __restrict__ dirty) {
    const int64_t b = blockIdx.x;
    const int t = threadIdx.x;
    if (b < npack) {
        const int64_t id = b * 256 + t;
        if (cin == cin_real && cout == cout_real) {
            pack_word<__bf16, false>(w, packed, 27, cin, cout,
                                     weight_strides(SPC_W_KRSC, 27, cin, cout), id);
            return;
        }
        // padded panels: word id holds 8 consecutive input channels of one
        // output channel (all real or all padding: both widths are
        // multiples of 8)
        using P = Panel<__bf16, false>;
        static_assert(P::G == 1, "one fragment per word");
        const int kch = cin / P::KC;
        const int ncol32 = cout / 32;
        if (id >= (int64_t)27 * kch * ncol32 * P::NG * 64) return;
        const int lane = (int)(id % 64);
        const int64_t rest = id / 64;
        const int g = (int)(rest % P::NG);
        const int64_t panel = rest / P::NG;
        const int c32 = (int)(panel % ncol32);
        const int64_t tk = panel / ncol32;
        const int kc = (int)(tk % kch);
        const int o = (int)(tk / kch);
        const int co = c32 * 32 + P::co_of(g, lane);
        const int ci0 = kc * P::KC + P::ci_of(g, lane);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (co < cout_real && ci0 < cin_real) {
            const uint16_t* src = reinterpret_cast<const uint16_t*>(w) +
                                  ((int64_t)co * 27 + o) * cin_real + ci0;
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (uint32_t)src[2 * e] | ((uint32_t)src[2 * e + 1] << 16);
            v = u32x4{h[0], h[1], h[2], h[3]};
        }
        packed[id] = v;
        return;
    }
    if (!cache) return;
    __shared__ int wd[27][4];
    const int64_t f2 = b - npack;
    const int64_t r = f2 * 256 + t;
    int32_t va[27], vc[27];
#pragma unroll
    for (int o = 0; o < 27; ++o) {
        va[o] = r < n ? idx[(int64_t)o * n + r] : 0;
        vc[o] = r < n ? cache[(int64_t)o * n + r] : 0;
    }
#pragma unroll
    for (int o = 0; o < 27; ++o) {
        const uint64_t bal = __ballot(va[o] != vc[o]);
        if ((t & 63) == 0) wd[o][t >> 6] = bal != 0;
    }
    __syncthreads();
    if (t < 54) {
        const int o = t % 27, h = t / 27;
        const int64_t f = 2 * f2 + h;
        if (f * 128 < n) dirty[f * 27 + o] = wd[o][2 * h] | wd[o][2 * h + 1];
    }
}

// Row copies between widths (16-bit elements, both widths multiples of 8):
// dst[r, c] = src[r, c] for c < min(cs, cd), zeros up to cd.  One thread
// per 16-byte piece of a destination row.
__global__ void bridge_copy_rows_kernel(const uint16_t* __restrict__ src, int64_t cs,
                                        uint16_t* __restrict__ dst, int64_t cd, int64_t rows) {
    const int64_t pr = cd / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * pr) return;
    const int64_t r = i / pr;
    const int64_t c = (i - r * pr) * 8;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (c < cs) {
        const uint16_t* p = src + r * cs + c;
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (uint32_t)p[2 * e] | ((uint32_t)p[2 * e + 1] << 16);
        v = u32x4{h[0], h[1], h[2], h[3]};
    }
    uint32_t* q = reinterpret_cast<uint32_t*>(dst + r * cd + c);
    q[0] = v.x;
    q[1] = v.y;
    q[2] = v.z;
    q[3] = v.w;
}

// The plan cache entry for n tokens (27 taps) and the tile geometry, from
// the device's four entries (the least recently used one replaced and
// reset: its copy then describes no plan tile), or null when it cannot be
// had (the call then runs without a plan).  Called with g_bridge_mu held.
BridgePlan* bridge_plan(BridgeDev& bd, hipStream_t s, int64_t n, int geometry) {
    BridgePlan* hit = nullptr;
    BridgePlan* lru = &bd.plans[0];
    for (BridgePlan& e : bd.plans) {
        if (e.n == n && e.geometry == geometry) hit = &e;
        if (e.used < lru->used) lru = &e;
    }
    ++bd.clock;
    if (hit) {
        hit->used = bd.clock;
        return hit;
    }
    BridgePlan& bp = *lru;
    bp.n = -1;
    bp.geometry = -1;
    bp.used = 0;
    const size_t need_idx = (size_t)(n + (n + 127) / 128) * 27 * sizeof(int32_t);
    const size_t need_plan = spc_conv_plan_bytes(n, 27);
    if (need_plan == 0) return nullptr;
    void* pi = bp.idx;
    if (!bridge_grow(pi, bp.idx_cap, need_idx)) {
        bp.idx = nullptr;
        return nullptr;
    }
    bp.idx = static_cast<int32_t*>(pi);
    if (!bridge_grow(bp.plan, bp.plan_cap, need_plan)) return nullptr;
    // entries no index equals: every tile of the first call sets itself up
    const int64_t ne = n * 27;
    fill_i32_kernel<<<(unsigned)ceil_div(ne, 256), 256, 0, s>>>(bp.idx, ne, INT_MIN);
    if (hipGetLastError() != hipSuccess) return nullptr;
    bp.dirty = bp.idx + n * 27;
    bp.n = n;
    bp.geometry = geometry;
    bp.used = bd.clock;
    return &bp;
}

// Tile-geometry override (spc_conv_set_tile_geometry; initially from
// SPC_CONV_GEOMETRY=wide / small / tall): 0 = each conv picks by shape.
std::atomic<int> g_geometry{[] {
    const char* e = getenv("SPC_CONV_GEOMETRY");
    if (e && strcmp(e, "wide") == 0) return SPC_TILES_WIDE;
    if (e && strcmp(e, "small") == 0) return SPC_TILES_SMALL;
    if (e && strcmp(e, "tall") == 0) return SPC_TILES_TALL;
    return SPC_TILES_AUTO;
}()};
int geometry_override() { return g_geometry.load(std::memory_order_relaxed); }

int check_shape(const char* fn, int64_t ntaps, int64_t cin, int64_t cout, bool any_taps = false) {
    const bool taps_ok = any_taps ? (ntaps >= 1 && ntaps <= 4096) : (ntaps == 27 || ntaps == 8 || ntaps == 1);
    if (!taps_ok || cin <= 0 || cout <= 0 || cin % 32 != 0 ||
        cout % 32 != 0 || cin > (1 << 16) || cout > (1 << 16) ||
        ntaps * cin * cout * 4 >= ((int64_t)1 << 31)) {
        set_last_error("%s: unsupported shape ntaps=%lld cin=%lld cout=%lld (ntaps 27, 8 or 1, "
                       "cin and cout multiples of 32, ntaps*cin*cout*4 below 2^31 bytes)",
                       fn, (long long)ntaps, (long long)cin, (long long)cout);
        return SPC_BAD_SHAPE;
    }
    return SPC_OK;
}

}  // namespace
}  // namespace spc

using namespace spc;

extern "C" {

size_t spc_conv_packed_bytes(int w_dtype, int64_t ntaps, int64_t cin, int64_t cout) {
    if (ntaps <= 0 || cin <= 0 || cout <= 0) return 0;
    switch (w_dtype) {
        case SPC_F32: return packed_quant_bytes<float, false>(ntaps, cin, cout);
        case SPC_F16:
        case SPC_BF16: return packed_quant_bytes<__bf16, false>(ntaps, cin, cout);
        case SPC_Q8_0:
            return align_up(packed_quant_bytes<__bf16, true>(ntaps, cin, cout), 256) +
                   (size_t)ntaps * (cin / 32) * cout * sizeof(float);
        default: return 0;
    }
}

int spc_conv_pack_weights(spc_stream_t stream, int w_dtype, int w_layout, const void* w,
                          const void* w_scale, int64_t ntaps, int64_t cin, int64_t cout,
                          void* packed) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    // any tap count: weight classes pack n_classes * ntaps taps
    const int st = check_shape("spc_conv_pack_weights", ntaps, cin, cout, true);
    if (st != SPC_OK) return st;
    if (!w || !packed || !aligned16(packed) || (w_dtype == SPC_Q8_0 && !w_scale)) {
        set_last_error("spc_conv_pack_weights: null / misaligned pointer");
        return SPC_BAD_ARG;
    }
    if (w_layout != SPC_W_KRSC && w_layout != SPC_W_TCK && w_layout != SPC_W_TKC) {
        set_last_error("spc_conv_pack_weights: unknown weight layout %d", w_layout);
        return SPC_BAD_ARG;
    }
    if (w_dtype == SPC_Q8_0 && w_layout == SPC_W_TKC) {
        set_last_error("spc_conv_pack_weights: Q8_0 blocks must run along cin (SPC_W_KRSC or "
                       "SPC_W_TCK); dequantise SPC_W_TKC weights first");
        return SPC_BAD_ARG;
    }
    const WStride ws = weight_strides(w_layout, ntaps, cin, cout);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    u32x4* out = static_cast<u32x4*>(packed);
    switch (w_dtype) {
        case SPC_F32: {
            const int64_t words = (int64_t)packed_quant_bytes<float, false>(ntaps, cin, cout) / 16;
            pack_weights_kernel<float, false><<<(unsigned)ceil_div(words, 256), 256, 0, s>>>(
                wb, out, (int)ntaps, (int)cin, (int)cout, ws);
            break;
        }
        case SPC_F16:
        case SPC_BF16: {
            const int64_t words = (int64_t)packed_quant_bytes<__bf16, false>(ntaps, cin, cout) / 16;
            pack_weights_kernel<__bf16, false><<<(unsigned)ceil_div(words, 256), 256, 0, s>>>(
                wb, out, (int)ntaps, (int)cin, (int)cout, ws);
            break;
        }
        case SPC_Q8_0: {
            const size_t qbytes = packed_quant_bytes<__bf16, true>(ntaps, cin, cout);
            const int64_t words = (int64_t)qbytes / 16;
            pack_weights_kernel<__bf16, true><<<(unsigned)ceil_div(words, 256), 256, 0, s>>>(
                wb, out, (int)ntaps, (int)cin, (int)cout, ws);
            float* sc = reinterpret_cast<float*>(static_cast<char*>(packed) + align_up(qbytes, 256));
            const int64_t ns = ntaps * (cin / 32) * cout;
            pack_scales_kernel<<<(unsigned)ceil_div(ns, 256), 256, 0, s>>>(
                static_cast<const uint16_t*>(w_scale), sc, (int)ntaps, (int)cin, (int)cout, ws);
            break;
        }
        default:
            set_last_error("spc_conv_pack_weights: unknown dtype %d", w_dtype);
            return SPC_BAD_ARG;
    }
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_conv_expand_q8_0(spc_stream_t stream, const void* packed_q8, int64_t ntaps, int64_t cin,
                         int64_t cout, void* packed_bf16) {
    return spc_conv_expand_q8_0_to(stream, packed_q8, ntaps, cin, cout, SPC_BF16, packed_bf16);
}

int spc_conv_expand_q8_0_to(spc_stream_t stream, const void* packed_q8, int64_t ntaps,
                            int64_t cin, int64_t cout, int out_dtype, void* packed_out) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = check_shape("spc_conv_expand_q8_0", ntaps, cin, cout, true);
    if (st != SPC_OK) return st;
    if (!packed_q8 || !packed_out || !aligned16(packed_q8) || !aligned16(packed_out) ||
        (out_dtype != SPC_BF16 && out_dtype != SPC_F16)) {
        set_last_error("spc_conv_expand_q8_0: null / misaligned pointer or out_dtype not "
                       "SPC_BF16 / SPC_F16");
        return SPC_BAD_ARG;
    }
    const size_t qbytes = packed_quant_bytes<__bf16, true>(ntaps, cin, cout);
    const int64_t panels = (int64_t)qbytes / 1024;
    const float* sc =
        reinterpret_cast<const float*>(static_cast<const char*>(packed_q8) + align_up(qbytes, 256));
    const unsigned grid = (unsigned)ceil_div(panels * 64, 256);
    if (out_dtype == SPC_F16)
        expand_q8_0_kernel<true><<<grid, 256, 0, s>>>(static_cast<const u32x4*>(packed_q8), sc,
                                                       static_cast<u32x4*>(packed_out), panels,
                                                       (int)(cout / 32), (int)cout);
    else
        expand_q8_0_kernel<false><<<grid, 256, 0, s>>>(static_cast<const u32x4*>(packed_q8), sc,
                                                        static_cast<u32x4*>(packed_out), panels,
                                                        (int)(cout / 32), (int)cout);
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_convert(spc_stream_t stream, int src_dtype, const void* src, int dst_dtype, void* dst,
                int64_t n) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto ok = [](int d) { return d == SPC_F32 || d == SPC_F16 || d == SPC_BF16; };
    if (n < 0 || !ok(src_dtype) || !ok(dst_dtype) || (n > 0 && (!src || !dst))) {
        set_last_error("spc_convert: bad arguments");
        return SPC_BAD_ARG;
    }
    if (n == 0) return SPC_OK;
    convert_kernel<<<(unsigned)ceil_div(ceil_div(n, 4), 256), 256, 0, s>>>(src, src_dtype, dst,
                                                                          dst_dtype, n);
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

size_t spc_conv_plan_bytes(int64_t n_out, int64_t ntaps) {
    if (n_out <= 0 || (ntaps != 27 && ntaps != 8 && ntaps != 1)) return 0;
    return (size_t)(plan_wide_bytes(n_out, (int)ntaps) + plan_small_bytes(n_out, (int)ntaps));
}

int spc_conv_plan(spc_stream_t stream, const int32_t* idx, int idx_layout,
                  const int32_t* row_perm, int64_t ntaps, int64_t n_out, int64_t n_in, void* plan,
                  size_t plan_bytes) {
    return spc_conv_plan_sections(stream, idx, idx_layout, row_perm, ntaps, n_out, n_in,
                                  SPC_PLAN_WIDE | SPC_PLAN_SMALL, plan, plan_bytes);
}

int spc_conv_plan_sections(spc_stream_t stream, const int32_t* idx, int idx_layout,
                           const int32_t* row_perm, int64_t ntaps, int64_t n_out, int64_t n_in,
                           uint32_t sections, void* plan, size_t plan_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if ((ntaps != 27 && ntaps != 8 && ntaps != 1) || n_out < 0 || n_in < 0 ||
        n_out > INT32_MAX || n_in > INT32_MAX) {
        set_last_error("spc_conv_plan: unsupported ntaps=%lld / n_out=%lld / n_in=%lld",
                       (long long)ntaps, (long long)n_out, (long long)n_in);
        return SPC_BAD_SHAPE;
    }
    if (n_out == 0) return SPC_OK;
    if ((!idx && (ntaps != 1 || n_in != n_out)) || !plan || ((uintptr_t)plan & 255u) != 0 ||
        (idx_layout != SPC_IDX_TOKEN_MAJOR && idx_layout != SPC_IDX_OFFSET_MAJOR) ||
        (sections & ~(SPC_PLAN_WIDE | SPC_PLAN_SMALL)) != 0) {
        set_last_error("spc_conv_plan: null / misaligned (256 bytes) pointer, bad layout or "
                       "unknown section bits");
        return SPC_BAD_ARG;
    }
    if (plan_bytes < spc_conv_plan_bytes(n_out, ntaps)) {
        set_last_error("spc_conv_plan: plan buffer too small");
        return SPC_OOM;
    }
    ConvArgs a{};
    a.idx = idx;
    a.row_perm = row_perm;
    a.n_out = n_out;
    a.n_in = n_in;
    a.idx_layout = idx_layout;
    a.ntaps = (int32_t)ntaps;
    // the wide tiles' plans, then the small tiles'; a section not asked for
    // has its tiles' markers cleared (its convs set their tiles up themselves)
    char* pl = static_cast<char*>(plan);
    char* ps = pl + plan_wide_bytes(n_out, (int)ntaps);
    auto section = [&](auto ntaps_c, auto geo_c, char* base, bool build) {
        constexpr int NT_ = decltype(ntaps_c)::value;
        using G = decltype(geo_c);
        const int64_t tiles = ceil_div(n_out, G::TM);
        if (build)
            conv_plan_kernel<NT_, G><<<(unsigned)tiles, 512, 0, s>>>(a, base);
        else
            plan_unmark_kernel<<<(unsigned)ceil_div(tiles, 256), 256, 0, s>>>(
                base, tiles, G::plan_tile_bytes(NT_));
    };
    const bool w = sections & SPC_PLAN_WIDE, sm = sections & SPC_PLAN_SMALL;
    if (ntaps == 27) {
        section(std::integral_constant<int, 27>{}, GeoWide{}, pl, w);
        section(std::integral_constant<int, 27>{}, GeoSmall<27>{}, ps, sm);
    } else if (ntaps == 8) {
        section(std::integral_constant<int, 8>{}, GeoWide{}, pl, w);
        section(std::integral_constant<int, 8>{}, GeoSmall<8>{}, ps, sm);
    } else {
        section(std::integral_constant<int, 1>{}, GeoWide{}, pl, w);
        section(std::integral_constant<int, 1>{}, GeoSmall<1>{}, ps, sm);
    }
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_sparse_conv(spc_stream_t stream, int dtype, const void* x, int w_dtype, int w_layout,
                    const void* w, const void* w_scale, const void* bias, void* y,
                    const int32_t* idx, int idx_layout, const int32_t* row_perm, int64_t ntaps,
                    int64_t n_out, int64_t n_in, int64_t cin, int64_t cout) {
    return spc_sparse_conv_plan(stream, dtype, x, w_dtype, w_layout, w, w_scale, bias, y, idx,
                                idx_layout, row_perm, nullptr, ntaps, n_out, n_in, cin, cout);
}

int spc_sparse_conv_plan(spc_stream_t stream, int dtype, const void* x, int w_dtype,
                         int w_layout, const void* w, const void* w_scale, const void* bias,
                         void* y, const int32_t* idx, int idx_layout, const int32_t* row_perm,
                         const void* plan, int64_t ntaps, int64_t n_out, int64_t n_in,
                         int64_t cin, int64_t cout) {
    return spc_sparse_conv_fused(stream, dtype, x, w_dtype, w_layout, w, w_scale, bias, y, idx,
                                 idx_layout, row_perm, plan, ntaps, n_out, n_in, cin, cout, nullptr);
}

namespace {

int conv_entry(spc_stream_t stream, int dtype, const void* x, int w_dtype, int w_layout,
               const void* w, const void* w_scale, const void* bias, void* y, const int32_t* idx,
               int idx_layout, const int32_t* row_perm, const void* plan, int64_t ntaps,
               int64_t n_out, int64_t n_in, int64_t cin, int64_t cout, int64_t class_rows,
               int64_t n_classes, const spc_conv_epilogue* epi, int32_t* idx_cache = nullptr,
               const int32_t* plan_dirty = nullptr) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = check_shape("spc_sparse_conv", ntaps, cin, cout);
    if (st != SPC_OK) return st;
    if (n_out < 0 || n_in < 0 || n_out > INT32_MAX || n_in > INT32_MAX) {
        set_last_error("spc_sparse_conv: n_out=%lld n_in=%lld out of range", (long long)n_out,
                       (long long)n_in);
        return SPC_BAD_SHAPE;
    }
    if (n_out == 0) return SPC_OK;
    if (!idx && (ntaps != 1 || n_in != n_out)) {
        set_last_error("spc_sparse_conv: idx may be NULL only for ntaps 1 with n_in == n_out");
        return SPC_BAD_ARG;
    }
    if (!x || !w || !y || !aligned16(x) || !aligned16(w) || !aligned16(y) ||
        (idx_layout != SPC_IDX_TOKEN_MAJOR && idx_layout != SPC_IDX_OFFSET_MAJOR) ||
        (w_layout != SPC_W_KRSC && w_layout != SPC_W_PACKED)) {
        set_last_error("spc_sparse_conv: null / misaligned pointer or bad layout enum");
        return SPC_BAD_ARG;
    }
    ConvArgs a{};
    a.x = x;
    a.w = w;
    a.wscale = w_scale;
    a.bias = bias;
    a.y = y;
    a.idx = idx;
    a.row_perm = row_perm;
    a.n_out = n_out;
    a.n_in = n_in;
    a.idx_layout = idx_layout;
    a.ntaps = (int32_t)ntaps;
    a.cin = (int32_t)cin;
    a.cout = (int32_t)cout;
    a.packed = w_layout == SPC_W_PACKED;
    if (class_rows > 0) {
        if (class_rows % GeoWide::TM != 0 || n_classes < 1 || n_classes * ntaps > 4096 ||
            n_classes * ntaps * cin * cout * 4 >= ((int64_t)1 << 31) ||
            n_out > class_rows * n_classes || !a.packed || w_dtype != dtype || w_dtype == SPC_Q8_0) {
            set_last_error("spc_sparse_conv_classes: class_rows must be a positive multiple of %d "
                           "with n_out <= class_rows * n_classes, weights packed in the feature "
                           "dtype (got class_rows=%lld n_classes=%lld n_out=%lld)",
                           GeoWide::TM, (long long)class_rows, (long long)n_classes, (long long)n_out);
            return SPC_BAD_ARG;
        }
        a.class_rows = class_rows;
        a.n_classes = (int32_t)n_classes;
    }
    if (plan && ((uintptr_t)plan & 255u) != 0) {
        set_last_error("spc_sparse_conv_plan: plan must be 256-byte aligned");
        return SPC_BAD_ARG;
    }
    a.plan = plan;
    if (idx_cache && (!plan || !plan_dirty || row_perm || !idx)) {
        set_last_error("spc_sparse_conv: a self-refreshing plan needs a plan, flags, idx and "
                       "natural row order");
        return SPC_BAD_ARG;
    }
    a.idx_cache = idx_cache;
    a.plan_dirty = plan_dirty;
    a.num_cu = device_cu_count();
    a.geometry = geometry_override();
    if (epi && epi->mode != SPC_EPI_NONE) {
        a.epi_mode = epi->mode;
        if (epi->mode == SPC_EPI_RESIDUAL) {
            if (!epi->residual || !aligned16(epi->residual)) {
                set_last_error("spc_sparse_conv_fused: residual must be a 16-byte aligned pointer");
                return SPC_BAD_ARG;
            }
            a.residual = epi->residual;
            if (epi->residual_rows) {
                if (epi->n_residual < 1 || epi->n_residual > INT32_MAX) {
                    set_last_error("spc_sparse_conv_fused: residual_rows needs 1 <= n_residual <= "
                                   "INT32_MAX (got %lld)", (long long)epi->n_residual);
                    return SPC_BAD_ARG;
                }
                a.residual_rows = epi->residual_rows;
                a.n_residual = epi->n_residual;
            }
        } else if (epi->mode == SPC_EPI_NORM_MOD_SILU) {
            // one tile must hold whole output rows with a power-of-two lane
            // group per row: widths 32, 64 and 128 (wider or other rows take
            // spc_layernorm_mod_silu after the conv)
            if (cout != 32 && cout != 64 && cout != 128) {
                set_last_error("spc_sparse_conv_fused: the norm epilogue needs cout 32, 64 or 128 "
                               "(got %lld)", (long long)cout);
                return SPC_BAD_SHAPE;
            }
            if (!epi->scale || !epi->shift || !epi->coords || !aligned16(epi->scale) ||
                !aligned16(epi->shift) || epi->n_batch < 1 || !(epi->eps >= 0.0f)) {
                set_last_error("spc_sparse_conv_fused: norm epilogue needs 16-byte aligned scale and "
                               "shift, coords, n_batch >= 1 and eps >= 0");
                return SPC_BAD_ARG;
            }
            a.epi_eps = epi->eps;
            a.epi_scale = epi->scale;
            a.epi_shift = epi->shift;
            a.coords = epi->coords;
            a.n_batch = epi->n_batch;
        } else {
            set_last_error("spc_sparse_conv_fused: unknown epilogue mode %d", epi->mode);
            return SPC_BAD_ARG;
        }
    }
    hipError_t e = hipSuccess;
    if (w_dtype == SPC_Q8_0) {
        if (dtype != SPC_BF16) {
            set_last_error("spc_sparse_conv: Q8_0 weights need bf16 activations");
            return SPC_BAD_ARG;
        }
        if (a.packed) {
            a.wscale = static_cast<const char*>(w) +
                       align_up(packed_quant_bytes<__bf16, true>(ntaps, cin, cout), 256);
        } else if (!w_scale) {
            set_last_error("spc_sparse_conv: Q8_0 weights in KRSC layout need w_scale");
            return SPC_BAD_ARG;
        }
        e = conv_q8(s, a);
    } else if (w_dtype != dtype) {
        set_last_error("spc_sparse_conv: w_dtype %d must equal dtype %d", w_dtype, dtype);
        return SPC_BAD_ARG;
    } else if (dtype == SPC_BF16) {
        e = conv_bf16(s, a);
    } else if (dtype == SPC_F16) {
        e = conv_f16(s, a);
    } else if (dtype == SPC_F32) {
        e = conv_f32(s, a);
    } else {
        set_last_error("spc_sparse_conv: unknown dtype %d", dtype);
        return SPC_BAD_ARG;
    }
    if (e != hipSuccess) return hip_status(e, "conv_kernel launch");
    return SPC_OK;
}

}  // namespace

int spc_sparse_conv_fused(spc_stream_t stream, int dtype, const void* x, int w_dtype,
                          int w_layout, const void* w, const void* w_scale, const void* bias,
                          void* y, const int32_t* idx, int idx_layout, const int32_t* row_perm,
                          const void* plan, int64_t ntaps, int64_t n_out, int64_t n_in,
                          int64_t cin, int64_t cout, const spc_conv_epilogue* epi) {
    return conv_entry(stream, dtype, x, w_dtype, w_layout, w, w_scale, bias, y, idx, idx_layout,
                      row_perm, plan, ntaps, n_out, n_in, cin, cout, 0, 1, epi);
}

int spc_sparse_conv_classes(spc_stream_t stream, int dtype, const void* x, const void* w,
                            const void* bias, void* y, const int32_t* idx, int idx_layout,
                            const int32_t* row_perm, const void* plan, int64_t ntaps,
                            int64_t n_out, int64_t n_in, int64_t cin, int64_t cout,
                            int64_t class_rows, int64_t n_classes, const spc_conv_epilogue* epi) {
    if (class_rows <= 0) {
        set_last_error("spc_sparse_conv_classes: class_rows must be positive");
        return SPC_BAD_ARG;
    }
    return conv_entry(stream, dtype, x, dtype, SPC_W_PACKED, w, nullptr, bias, y, idx, idx_layout,
                      row_perm, plan, ntaps, n_out, n_in, cin, cout, class_rows, n_classes, epi);
}

int spc_conv_tile_geometry(int dtype, int w_dtype, int64_t ntaps, int64_t n_out, int64_t cin,
                           int64_t cout, int64_t class_rows, int epi_mode) {
    ConvArgs a{};
    a.n_out = n_out;
    a.ntaps = (int32_t)ntaps;
    a.cin = (int32_t)cin;
    a.cout = (int32_t)cout;
    a.class_rows = class_rows;
    a.epi_mode = epi_mode;
    a.num_cu = device_cu_count();
    a.geometry = geometry_override();
    int g = SPC_TILES_WIDE;
    auto pick = [&](auto t_c, auto q8_c) {
        using T = decltype(t_c);
        constexpr bool Q8 = decltype(q8_c)::value;
        if (ntaps == 27 && use_tall_tiles<T, Q8, true, 27>(a)) g = SPC_TILES_TALL;
        else if (ntaps == 27 && use_small_tiles<T, Q8, true, 27>(a)) g = SPC_TILES_SMALL;
        else if (ntaps == 8 && use_small_tiles<T, Q8, true, 8>(a)) g = SPC_TILES_SMALL;
    };
    if (w_dtype == SPC_Q8_0) pick(__bf16{}, std::true_type{});
    else if (dtype == SPC_F32) pick(float{}, std::false_type{});
    else pick(__bf16{}, std::false_type{});  // bf16 and f16: 2-byte rows
    return g;
}

int spc_conv_set_tile_geometry(int geometry) {
    if (geometry != SPC_TILES_AUTO && geometry != SPC_TILES_WIDE && geometry != SPC_TILES_SMALL &&
        geometry != SPC_TILES_TALL) {
        set_last_error("spc_conv_set_tile_geometry: unknown geometry %d", geometry);
        return SPC_BAD_ARG;
    }
    g_geometry.store(geometry, std::memory_order_relaxed);
    return SPC_OK;
}

void sam3d_spconv_f16_forward(spc_stream_t stream, const void* input, const void* weight,
                              const void* bias, void* output, const int32_t* indices,
                              const uint32_t* mask, const int32_t* mask_argsort, int64_t tokens,
                              int64_t channels, int64_t output_channels) {
    // each tile's tap set is formed from the indices themselves, and rows run
    // in natural order (spatially coherent tiles share their gathered rows);
    // every output row is computed the same way in any order
    (void)mask;
    (void)mask_argsort;
    clear_last_error();  // spc_last_error() reports this call only
    // channel widths in multiples of 8, as the reference's spconv iterators
    // take them (ForwardDgradSparseIOIterator.h:58-61); widths that are not
    // multiples of 32 run zero-padded to the next multiple of 32
    if (channels <= 0 || output_channels <= 0 || channels % 8 != 0 || output_channels % 8 != 0 ||
        channels > (1 << 16) || output_channels > (1 << 16) || tokens < 0 || tokens > INT32_MAX) {
        set_last_error("sam3d_spconv_f16_forward: unsupported shape tokens=%lld channels=%lld "
                       "output_channels=%lld (channel widths multiples of 8, at most 65536)",
                       (long long)tokens, (long long)channels, (long long)output_channels);
        return;
    }
    const int64_t cin = (channels + 31) / 32 * 32;
    const int64_t cout = (output_channels + 31) / 32 * 32;
    if (check_shape("sam3d_spconv_f16_forward", 27, cin, cout) != SPC_OK) return;
    if (tokens == 0) return;
    if (!input || !weight || !output || !indices || !aligned16(input) || !aligned16(output)) {
        set_last_error("sam3d_spconv_f16_forward: null or misaligned (16 bytes) pointer");
        return;
    }
    const bool padded = cin != channels || cout != output_channels;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        set_last_error("sam3d_spconv_f16_forward: no current device");
        return;
    }
    std::lock_guard<std::mutex> lock(g_bridge_mu);
    BridgeDev& bd = g_bridge[dev];
    // The weights arrive in KRSC order on every call (the ggml shim passes
    // its weight tensor).  Packed into the MFMA fragment order first, each
    // B operand is one contiguous 1 KB load instead of 32 strided 32-byte
    // pieces: one pack kernel (weight bytes read and written once) buys the
    // packed conv.
    const size_t wbytes = spc_conv_packed_bytes(SPC_F16, 27, cin, cout);
    if (!bridge_grow(bd.pack, bd.pack_cap, wbytes)) {
        set_last_error("sam3d_spconv_f16_forward: cannot allocate %zu bytes for the packed "
                       "weights", wbytes);
        return;
    }
    // padded widths: input, bias and output copies in one held buffer
    const void* xin = input;
    const void* bin = bias;
    void* yout = output;
    if (padded) {
        const size_t xb = cin != channels ? align_up((size_t)tokens * cin * 2, 256) : 0;
        const size_t yb = cout != output_channels ? align_up((size_t)tokens * cout * 2, 256) : 0;
        const size_t bb = align_up((size_t)cout * 2, 256);
        if (!bridge_grow(bd.pad, bd.pad_cap, xb + yb + bb)) {
            set_last_error("sam3d_spconv_f16_forward: cannot allocate %zu bytes for the padded "
                           "rows", xb + yb + bb);
            return;
        }
        char* pb = static_cast<char*>(bd.pad);
        uint16_t* bpad = reinterpret_cast<uint16_t*>(pb + xb + yb);
        if (cin != channels) {
            bridge_copy_rows_kernel<<<(unsigned)ceil_div(tokens * cin / 8, 256), 256, 0, s>>>(
                static_cast<const uint16_t*>(input), channels, reinterpret_cast<uint16_t*>(pb), cin,
                tokens);
            xin = pb;
        }
        if (cout != output_channels) yout = pb + xb;
        if (bias && cout != output_channels) {
            bridge_copy_rows_kernel<<<1, 256, 0, s>>>(static_cast<const uint16_t*>(bias),
                                                      output_channels, bpad, cout, 1);
            bin = bpad;
        }
        if (hipGetLastError() != hipSuccess) {
            set_last_error("sam3d_spconv_f16_forward: padding launch failed");
            return;
        }
    }
    // The tile setup (the deduplicated gather of each tile) comes from the
    // device's self-refreshing plans: built by the first call over an index
    // table, reused by every later call over the same one.
    const int geometry = spc_conv_tile_geometry(SPC_F16, SPC_F16, 27, tokens, cin, cout, 0,
                                                SPC_EPI_NONE);
    BridgePlan* bp = bridge_plan(bd, s, tokens, geometry);
    const void* plan = bp ? bp->plan : nullptr;
    int32_t* cache = bp ? bp->idx : nullptr;
    const int32_t* dirty = bp ? bp->dirty : nullptr;
    // one launch packs the weights and flags the changed index entries
    const int64_t npack = (int64_t)(wbytes / 16 + 255) / 256;
    const int64_t nflag = bp ? (tokens + 255) / 256 : 0;
    bridge_prep_kernel<<<(unsigned)(npack + nflag), 256, 0, s>>>(
        static_cast<const uint8_t*>(weight), static_cast<u32x4*>(bd.pack), (int)cin, (int)cout,
        (int)channels, (int)output_channels, npack, indices, cache, tokens,
        bp ? bp->dirty : nullptr);
    if (hipGetLastError() != hipSuccess) {
        set_last_error("sam3d_spconv_f16_forward: preparation launch failed");
        return;
    }
    if (conv_entry(stream, SPC_F16, xin, SPC_F16, SPC_W_PACKED, bd.pack, nullptr, bin, yout,
                   indices, SPC_IDX_OFFSET_MAJOR, nullptr, plan, 27, tokens, tokens, cin, cout, 0,
                   1, nullptr, cache, dirty) != SPC_OK)
        return;
    if (yout != output) {
        // padded output width: the first output_channels columns
        bridge_copy_rows_kernel<<<(unsigned)ceil_div(tokens * output_channels / 8, 256), 256, 0, s>>>(
            static_cast<const uint16_t*>(yout), cout, static_cast<uint16_t*>(output), output_channels,
            tokens);
        if (hipGetLastError() != hipSuccess)
            set_last_error("sam3d_spconv_f16_forward: output copy launch failed");
    }
}

int spc_q8_0_repack(spc_stream_t stream, const uint8_t* blocks, int64_t nblocks, int8_t* qs,
                    uint16_t* d) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (nblocks < 0 || !blocks || !qs || !d || !aligned16(qs)) {
        set_last_error("spc_q8_0_repack: bad arguments");
        return SPC_BAD_ARG;
    }
    if (nblocks == 0) return SPC_OK;
    q8_0_repack_kernel<<<(unsigned)ceil_div(nblocks, 256), 256, 0, s>>>(blocks, nblocks, qs, d);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "q8_0_repack launch");
    return SPC_OK;
}

int spc_q8_0_quantize(spc_stream_t stream, const float* w, int64_t n, uint8_t* blocks) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n < 0 || n % 32 != 0 || (n > 0 && (!w || !blocks || !aligned16(w)))) {
        set_last_error("spc_q8_0_quantize: n must be a multiple of 32, w 16-byte aligned");
        return SPC_BAD_ARG;
    }
    if (n == 0) return SPC_OK;
    const int64_t nb = n / 32;
    q8_0_quantize_kernel<<<(unsigned)ceil_div(nb, 256), 256, 0, s>>>(w, nb, blocks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "q8_0_quantize launch");
    return SPC_OK;
}

int spc_q8_0_dequant(spc_stream_t stream, const uint8_t* blocks, int64_t nblocks, int out_dtype,
                     void* out) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (nblocks < 0 || (nblocks > 0 && (!blocks || !out)) ||
        (out_dtype != SPC_F32 && out_dtype != SPC_F16 && out_dtype != SPC_BF16)) {
        set_last_error("spc_q8_0_dequant: bad arguments");
        return SPC_BAD_ARG;
    }
    if (nblocks == 0) return SPC_OK;
    const int64_t n = nblocks * 32;
    q8_0_dequant_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, s>>>(blocks, n, out_dtype, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "q8_0_dequant launch");
    return SPC_OK;
}

}  // extern "C"
