// scatter.hip -- feature ops on the downsample / upsample / subdivide maps.
//
//   spc_scatter_mean : deterministic scatter-mean with the ggml CPU op's
//                      rounding history (PATCH:151-215): fine rows grouped
//                      by destination with a stable radix sort (ascending
//                      fine row inside a group), then one thread per
//                      (coarse row, channel) adds in that order, rounding the
//                      partial sum to the storage dtype after every add, and
//                      divides by the count in F32 (16-byte groups of
//                      channels per thread where the rows allow).
//   spc_children_mean: the same values from the downsample map's children
//                      lists (ascending fine rows, at most 8 per coarse row):
//                      no sort, one pass.
//   spc_gather_rows  : dst[i] = src[idx[i]] with 16-byte vector copies.
#include "common.h"

namespace spc {

namespace {

__global__ void scatter_keys_kernel(const int32_t* __restrict__ rows, int64_t nf, int64_t nc,
                                    uint32_t* __restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nf) return;
    const int32_t r = rows[i];
    keys[i] = (r >= 0 && r < nc) ? (uint32_t)r : (uint32_t)nc;
}

// seg[r] = first sorted position whose key >= r, for r in [0, nc]
__global__ void segment_bounds_kernel(const uint32_t* __restrict__ sk, int64_t nf, int64_t nc,
                                      int32_t* __restrict__ seg) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > nc) return;
    int64_t lo = 0, hi = nf;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)sk[mid] < r) lo = mid + 1;
        else hi = mid;
    }
    seg[r] = (int32_t)lo;
}

template <int DT>
struct Store;
template <>
struct Store<SPC_F16> {
    typedef uint16_t t;
    __device__ static float ld(t v) { return f16_bits_to_f32(v); }
    __device__ static t st(float v) { return f32_to_f16_bits(v); }
};
template <>
struct Store<SPC_BF16> {
    typedef uint16_t t;
    __device__ static float ld(t v) { return bf16_bits_to_f32(v); }
    __device__ static t st(float v) { return f32_to_bf16_bits(v); }
};
template <>
struct Store<SPC_F32> {
    typedef float t;
    __device__ static float ld(t v) { return v; }
    __device__ static t st(float v) { return v; }
};

template <int DT>
__global__ __launch_bounds__(256) void scatter_mean_kernel(
    const typename Store<DT>::t* __restrict__ feats, const int32_t* __restrict__ sv,
    const int32_t* __restrict__ seg, const float* __restrict__ counts, int64_t channels,
    int64_t nc, typename Store<DT>::t* __restrict__ out) {
    using S = Store<DT>;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nc * channels) return;
    const int64_t r = e / channels;
    const int64_t c = e - r * channels;
    typename S::t acc = S::st(0.0f);
    const int32_t b = seg[r];
    const int32_t end = seg[r + 1];
    for (int32_t p = b; p < end; ++p) acc = S::st(S::ld(acc) + S::ld(feats[(int64_t)sv[p] * channels + c]));
    out[e] = S::st(S::ld(acc) / counts[r]);
}

// scatter_mean_kernel over 16-byte groups of channels (channels a multiple
// of the group): one thread per (coarse row, group), the adds per element
// in the same order.
template <int DT>
__global__ __launch_bounds__(256) void scatter_mean_vec_kernel(
    const u32x4* __restrict__ feats, const int32_t* __restrict__ sv,
    const int32_t* __restrict__ seg, const float* __restrict__ counts, int64_t groups,
    int64_t nc, u32x4* __restrict__ out) {
    using S = Store<DT>;
    using T = typename S::t;
    constexpr int VEC = 16 / sizeof(T);
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nc * groups) return;
    const int64_t r = e / groups;
    const int64_t q = e - r * groups;
    T acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = S::st(0.0f);
    const int32_t b = seg[r];
    const int32_t end = seg[r + 1];
    for (int32_t p = b; p < end; ++p) {
        const u32x4 w = feats[(int64_t)sv[p] * groups + q];
        T x[VEC];
        __builtin_memcpy(x, &w, 16);
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = S::st(S::ld(acc[v]) + S::ld(x[v]));
    }
    const float cnt = counts[r];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = S::st(S::ld(acc[v]) / cnt);
    u32x4 o;
    __builtin_memcpy(&o, acc, 16);
    out[e] = o;
}

// The scatter-mean of one (coarse row, channel) from its children list
// (ascending fine rows, padded with values outside [0, nf)): the same adds
// in the same order as scatter_mean_kernel over the sorted rows.
template <int DT>
__global__ __launch_bounds__(256) void children_mean_kernel(
    const typename Store<DT>::t* __restrict__ feats, const int32_t* __restrict__ children,
    const float* __restrict__ counts, int64_t channels, int64_t nf, int64_t nc,
    typename Store<DT>::t* __restrict__ out) {
    using S = Store<DT>;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nc * channels) return;
    const int64_t r = e / channels;
    const int64_t c = e - r * channels;
    typename S::t acc = S::st(0.0f);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int32_t f = children[r * 8 + k];
        if (f < 0 || f >= nf) break;  // compacted lists: the padding ends them
        acc = S::st(S::ld(acc) + S::ld(feats[(int64_t)f * channels + c]));
    }
    out[e] = S::st(S::ld(acc) / counts[r]);
}

// The same over 16-byte groups of channels (channels a multiple of the
// group): one thread per (coarse row, group), 16-byte loads and stores, the
// adds per element as above.
template <int DT>
__global__ __launch_bounds__(256) void children_mean_vec_kernel(
    const u32x4* __restrict__ feats, const int32_t* __restrict__ children,
    const float* __restrict__ counts, int64_t groups, int64_t nf, int64_t nc,
    u32x4* __restrict__ out) {
    using S = Store<DT>;
    using T = typename S::t;
    constexpr int VEC = 16 / sizeof(T);
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nc * groups) return;
    const int64_t r = e / groups;
    const int64_t q = e - r * groups;
    T acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = S::st(0.0f);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int32_t f = children[r * 8 + k];
        if (f < 0 || f >= nf) break;
        const u32x4 w = feats[(int64_t)f * groups + q];
        T x[VEC];
        __builtin_memcpy(x, &w, 16);
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = S::st(S::ld(acc[v]) + S::ld(x[v]));
    }
    const float cnt = counts[r];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = S::st(S::ld(acc[v]) / cnt);
    u32x4 o;
    __builtin_memcpy(&o, acc, 16);
    out[e] = o;
}

template <typename V>
__global__ void gather_rows_kernel(const V* __restrict__ src, const int32_t* __restrict__ idx,
                                   V* __restrict__ dst, int64_t n_out, int64_t n_src,
                                   int64_t vec_per_row) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_out * vec_per_row) return;
    const int64_t i = e / vec_per_row;
    const int64_t v = e - i * vec_per_row;
    const int32_t s = idx[i];
    V val;
    if (s >= 0 && s < n_src) {
        val = src[(int64_t)s * vec_per_row + v];
    } else {
        val = V{};
    }
    dst[e] = val;
}

inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

int bits_for(int64_t v) {
    int b = 0;
    while (b < 62 && (1ll << b) < v) ++b;
    return b;
}

}  // namespace
}  // namespace spc

using namespace spc;

extern "C" {

size_t spc_scatter_mean_workspace_bytes(int64_t nf, int64_t nc) {
    const int64_t n = nf > 0 ? nf : 1;
    Sizer z;
    z.take<uint32_t>(n);
    z.take<uint32_t>(n);
    z.take<int32_t>(n);
    z.take<int32_t>((nc > 0 ? nc : 0) + 1);
    z.take<char>(radix_sort_ws_bytes(n, 4));
    return z.used + 256;
}

int spc_scatter_mean(spc_stream_t stream, int dtype, const void* features, const int32_t* rows,
                     const float* counts, void* out, int64_t channels, int64_t nf, int64_t nc,
                     void* workspace, size_t workspace_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (channels <= 0 || nf < 0 || nc < 0 || nf > INT32_MAX || nc >= INT32_MAX) {
        set_last_error("spc_scatter_mean: bad shape");
        return SPC_BAD_SHAPE;
    }
    if (nc == 0) return SPC_OK;
    if (!out || !counts || (nf > 0 && (!features || !rows)) || !workspace) {
        set_last_error("spc_scatter_mean: null argument");
        return SPC_BAD_ARG;
    }
    const int64_t n = nf > 0 ? nf : 1;
    Carver c(workspace, workspace_bytes);
    uint32_t* keys = c.take<uint32_t>(n);
    uint32_t* sk = c.take<uint32_t>(n);
    int32_t* sv = c.take<int32_t>(n);
    int32_t* seg = c.take<int32_t>(nc + 1);
    const size_t sort_bytes = radix_sort_ws_bytes(n, 4);
    char* sort_ws = c.take<char>(sort_bytes);
    if (!c.ok) {
        set_last_error("spc_scatter_mean: workspace too small");
        return SPC_OOM;
    }
    if (nf > 0) {
        scatter_keys_kernel<<<grid_for(nf, 256), 256, 0, s>>>(rows, nf, nc, keys);
        SPC_HIP(radix_sort_u32(s, keys, nullptr, sk, sv, nf, bits_for(nc + 1), sort_ws,
                               sort_bytes));
    }
    segment_bounds_kernel<<<grid_for(nc + 1, 256), 256, 0, s>>>(sk, nf, nc, seg);
    const int es = dtype == SPC_F32 ? 4 : 2;
    if ((dtype == SPC_F16 || dtype == SPC_BF16 || dtype == SPC_F32) && channels * es % 16 == 0 &&
        ((uintptr_t)features & 15u) == 0 && ((uintptr_t)out & 15u) == 0) {
        const int64_t groups = channels * es / 16;
        const unsigned gv = grid_for(nc * groups, 256);
        const u32x4* fv = static_cast<const u32x4*>(features);
        u32x4* ov = static_cast<u32x4*>(out);
        if (dtype == SPC_F16)
            scatter_mean_vec_kernel<SPC_F16><<<gv, 256, 0, s>>>(fv, sv, seg, counts, groups, nc, ov);
        else if (dtype == SPC_BF16)
            scatter_mean_vec_kernel<SPC_BF16><<<gv, 256, 0, s>>>(fv, sv, seg, counts, groups, nc, ov);
        else
            scatter_mean_vec_kernel<SPC_F32><<<gv, 256, 0, s>>>(fv, sv, seg, counts, groups, nc, ov);
        SPC_HIP(hipGetLastError());
        return SPC_OK;
    }
    const unsigned g = grid_for(nc * channels, 256);
    switch (dtype) {
        case SPC_F16:
            scatter_mean_kernel<SPC_F16><<<g, 256, 0, s>>>(
                static_cast<const uint16_t*>(features), sv, seg, counts, channels, nc,
                static_cast<uint16_t*>(out));
            break;
        case SPC_BF16:
            scatter_mean_kernel<SPC_BF16><<<g, 256, 0, s>>>(
                static_cast<const uint16_t*>(features), sv, seg, counts, channels, nc,
                static_cast<uint16_t*>(out));
            break;
        case SPC_F32:
            scatter_mean_kernel<SPC_F32><<<g, 256, 0, s>>>(static_cast<const float*>(features),
                                                           sv, seg, counts, channels, nc,
                                                           static_cast<float*>(out));
            break;
        default:
            set_last_error("spc_scatter_mean: unknown dtype %d", dtype);
            return SPC_BAD_ARG;
    }
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_children_mean(spc_stream_t stream, int dtype, const void* features,
                      const int32_t* children, const float* counts, void* out, int64_t channels,
                      int64_t nf, int64_t nc) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (channels <= 0 || nf < 0 || nc < 0 || nf > INT32_MAX || nc >= INT32_MAX) {
        set_last_error("spc_children_mean: bad shape");
        return SPC_BAD_SHAPE;
    }
    if (nc == 0) return SPC_OK;
    if (!out || !counts || !children || (nf > 0 && !features)) {
        set_last_error("spc_children_mean: null argument");
        return SPC_BAD_ARG;
    }
    const int es = dtype == SPC_F32 ? 4 : 2;
    const bool vec = channels * es % 16 == 0 && ((uintptr_t)features & 15u) == 0 &&
                     ((uintptr_t)out & 15u) == 0;
    if (vec && (dtype == SPC_F16 || dtype == SPC_BF16 || dtype == SPC_F32)) {
        const int64_t groups = channels * es / 16;
        const unsigned gv = grid_for(nc * groups, 256);
        const u32x4* fv = static_cast<const u32x4*>(features);
        u32x4* ov = static_cast<u32x4*>(out);
        if (dtype == SPC_F16)
            children_mean_vec_kernel<SPC_F16><<<gv, 256, 0, s>>>(fv, children, counts, groups, nf, nc, ov);
        else if (dtype == SPC_BF16)
            children_mean_vec_kernel<SPC_BF16><<<gv, 256, 0, s>>>(fv, children, counts, groups, nf, nc, ov);
        else
            children_mean_vec_kernel<SPC_F32><<<gv, 256, 0, s>>>(fv, children, counts, groups, nf, nc, ov);
        SPC_HIP(hipGetLastError());
        return SPC_OK;
    }
    const unsigned g = grid_for(nc * channels, 256);
    switch (dtype) {
        case SPC_F16:
            children_mean_kernel<SPC_F16><<<g, 256, 0, s>>>(
                static_cast<const uint16_t*>(features), children, counts, channels, nf, nc,
                static_cast<uint16_t*>(out));
            break;
        case SPC_BF16:
            children_mean_kernel<SPC_BF16><<<g, 256, 0, s>>>(
                static_cast<const uint16_t*>(features), children, counts, channels, nf, nc,
                static_cast<uint16_t*>(out));
            break;
        case SPC_F32:
            children_mean_kernel<SPC_F32><<<g, 256, 0, s>>>(static_cast<const float*>(features),
                                                            children, counts, channels, nf, nc,
                                                            static_cast<float*>(out));
            break;
        default:
            set_last_error("spc_children_mean: unknown dtype %d", dtype);
            return SPC_BAD_ARG;
    }
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_gather_rows(spc_stream_t stream, int dtype, const void* src, const int32_t* idx,
                    void* dst, int64_t n_out, int64_t n_src, int64_t channels) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_out < 0 || n_src < 0 || channels <= 0) {
        set_last_error("spc_gather_rows: bad shape");
        return SPC_BAD_SHAPE;
    }
    if (n_out == 0) return SPC_OK;
    if (!src || !idx || !dst) {
        set_last_error("spc_gather_rows: null argument");
        return SPC_BAD_ARG;
    }
    int64_t es;
    switch (dtype) {
        case SPC_F32: es = 4; break;
        case SPC_F16:
        case SPC_BF16: es = 2; break;
        default:
            set_last_error("spc_gather_rows: unknown dtype %d", dtype);
            return SPC_BAD_ARG;
    }
    const int64_t row_bytes = channels * es;
    const bool a16 = ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
    const bool a4 = ((uintptr_t)src % 4 == 0) && ((uintptr_t)dst % 4 == 0);
    if (row_bytes % 16 == 0 && a16) {
        const int64_t v = row_bytes / 16;
        gather_rows_kernel<uint4><<<grid_for(n_out * v, 256), 256, 0, s>>>(
            static_cast<const uint4*>(src), idx, static_cast<uint4*>(dst), n_out, n_src, v);
    } else if (row_bytes % 4 == 0 && a4) {
        const int64_t v = row_bytes / 4;
        gather_rows_kernel<uint32_t><<<grid_for(n_out * v, 256), 256, 0, s>>>(
            static_cast<const uint32_t*>(src), idx, static_cast<uint32_t*>(dst), n_out, n_src, v);
    } else {
        const int64_t v = row_bytes / 2;
        gather_rows_kernel<uint16_t><<<grid_for(n_out * v, 256), 256, 0, s>>>(
            static_cast<const uint16_t*>(src), idx, static_cast<uint16_t*>(dst), n_out, n_src, v);
    }
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

}  // extern "C"
