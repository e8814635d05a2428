// norm.hip -- row LayerNorm + SiLU over [n, c] features: the prologue of the
// SLAT sparse residual block (structured_latent_flow.py:66-67: norm1 ->
// F.silu; native graph SRC/slat_flow_graph.cpp:331-341).
//
// Each row is handled by G = min(64, c / 4) lanes of a wave (64 / G rows
// per wave), every lane holding runs of 4 consecutive channels (one 8- or
// 16-byte load).  Mean and biased variance are formed in F32 with two
// passes over the registers and group-local shuffles.
#include <algorithm>

#include "common.h"

namespace spc {

namespace {

constexpr int kNormMaxC = 2048;

template <int DT>
struct Elem;  // feature loads / stores (streaming outputs: non-temporal stores)
template <>
struct Elem<SPC_F32> {
    __device__ static void ld4(const void* p, int64_t i, float* v) {
        const floatx4 q = *reinterpret_cast<const floatx4*>(static_cast<const float*>(p) + i);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
    __device__ static void st4(void* p, int64_t i, const float* v) {
        __builtin_nontemporal_store(floatx4{v[0], v[1], v[2], v[3]},
                                    reinterpret_cast<floatx4*>(static_cast<float*>(p) + i));
    }
    __device__ static float round(float v) { return v; }
};
template <>
struct Elem<SPC_BF16> {
    __device__ static void ld4(const void* p, int64_t i, float* v) {
        const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + i);
        v[0] = __uint_as_float(q.x << 16); v[1] = __uint_as_float(q.x & 0xffff0000u);
        v[2] = __uint_as_float(q.y << 16); v[3] = __uint_as_float(q.y & 0xffff0000u);
    }
    __device__ static void st4(void* p, int64_t i, const float* v) {
        __builtin_nontemporal_store(
            u32x2{(uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16),
                  (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16)},
            reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i));
    }
    __device__ static float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
};
template <>
struct Elem<SPC_F16> {
    __device__ static void ld4(const void* p, int64_t i, float* v) {
        const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + i);
        v[0] = f16_bits_to_f32((uint16_t)q.x); v[1] = f16_bits_to_f32((uint16_t)(q.x >> 16));
        v[2] = f16_bits_to_f32((uint16_t)q.y); v[3] = f16_bits_to_f32((uint16_t)(q.y >> 16));
    }
    __device__ static void st4(void* p, int64_t i, const float* v) {
        __builtin_nontemporal_store(
            u32x2{(uint32_t)f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16),
                  (uint32_t)f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16)},
            reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i));
    }
    __device__ static float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
};

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Per-batch modulation after the norm (SparseResBlock3d's `norm2(h) * (1 +
// scale) + shift`, structured_latent_flow.py:70): scale / shift f32
// [n_batch, c] holding feature-dtype values, the row's batch b = coords[4 t]
// (clamped to [0, n_batch)).
struct NormMod {
    const float* scale;
    const float* shift;
    const int32_t* coords;
    int64_t n_batch;
};

// G lanes per row, NV runs of 4 per lane (c <= 4 * G * NV), R rows per lane
// group (rows r, r + groups, ...: R independent reductions in flight)
template <int DT, int G, int NV, int R>
__global__ __launch_bounds__(256) void layernorm_silu_kernel(const void* __restrict__ x, int64_t n,
                                                             int c, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             float eps, int silu,
                                                             void* __restrict__ y, NormMod mod) {
    using E = Elem<DT>;
    const int lane = threadIdx.x & 63;
    constexpr int GPB = 256 / G;  // row groups per block
    const int64_t row0 = (int64_t)blockIdx.x * GPB * R + threadIdx.x / G;
    const int gl = lane % G;      // lane within the row's group
    float v[R][NV][4];
    float gv[NV][4], bv[NV][4];
    float s[R], q[R];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c0 = 4 * (gl + G * k);
        const bool in = c0 < c;
        const floatx4 g4 = gamma && in ? *reinterpret_cast<const floatx4*>(gamma + c0)
                                       : floatx4{1.f, 1.f, 1.f, 1.f};
        const floatx4 b4 = beta && in ? *reinterpret_cast<const floatx4*>(beta + c0)
                                      : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            gv[k][e] = g4[e];
            bv[k][e] = b4[e];
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = row0 + (int64_t)r * GPB;
        s[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c0 = 4 * (gl + G * k);
            if (row < n && c0 < c) E::ld4(x, row * c + c0, v[r][k]);
            else v[r][k][0] = v[r][k][1] = v[r][k][2] = v[r][k][3] = 0.0f;
            s[r] += (v[r][k][0] + v[r][k][1]) + (v[r][k][2] + v[r][k][3]);
        }
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < R; ++r) s[r] += __shfl_xor(s[r], off);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float mean = s[r] / (float)c;
        q[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (4 * (gl + G * k) < c) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[r][k][e] -= mean;
                    q[r] += v[r][k][e] * v[r][k][e];
                }
            }
        }
    }
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] += __shfl_xor(q[r], off);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = row0 + (int64_t)r * GPB;
        if (row >= n) continue;
        const float rstd = 1.0f / sqrtf(q[r] / (float)c + eps);
        const float* msc = nullptr;
        const float* msh = nullptr;
        if (mod.scale) {
            const int64_t b = min(max((int64_t)mod.coords[row * 4], (int64_t)0), mod.n_batch - 1);
            msc = mod.scale + b * c;
            msh = mod.shift + b * c;
        }
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c0 = 4 * (gl + G * k);
            if (c0 >= c) continue;
            float o[4];
            floatx4 sc4 = {0.f, 0.f, 0.f, 0.f}, sh4 = {0.f, 0.f, 0.f, 0.f};
            if (msc) {
                sc4 = *reinterpret_cast<const floatx4*>(msc + c0);
                sh4 = *reinterpret_cast<const floatx4*>(msh + c0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float u = v[r][k][e] * rstd;
                if (gamma) u *= gv[k][e];
                if (beta) u += bv[k][e];
                u = E::round(u);  // LayerNorm32 casts back to the feature dtype
                if (msc)          // * (1 + scale) + shift, each op rounded to the dtype
                    u = E::round(E::round(u * E::round(1.0f + sc4[e])) + sh4[e]);
                if (silu) u = silu_f32(u);
                o[e] = u;
            }
            E::st4(y, row * c + c0, o);
        }
    }
}

template <int DT, int G, int NV, int R>
void launch_g(hipStream_t s, const void* x, int64_t n, int c, const float* gamma, const float* beta,
              float eps, int silu, void* y, const NormMod& mod) {
    const dim3 grid((unsigned)ceil_div(n, (int64_t)(256 / G) * R));
    layernorm_silu_kernel<DT, G, NV, R><<<grid, dim3(256), 0, s>>>(x, n, c, gamma, beta, eps, silu,
                                                                   y, mod);
}

template <int DT>
hipError_t launch_norm(hipStream_t s, const void* x, int64_t n, int c, const float* gamma,
                       const float* beta, float eps, int silu, void* y, const NormMod& mod) {
    const int runs = c / 4;
    if (runs <= 64) {
        // G = smallest power of two >= runs: several rows per wave
        int g = 1;
        while (g < runs) g <<= 1;
        switch (g) {
            case 1: launch_g<DT, 1, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
            case 2: launch_g<DT, 2, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
            case 4: launch_g<DT, 4, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
            case 8: launch_g<DT, 8, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
            case 16: launch_g<DT, 16, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
            case 32: launch_g<DT, 32, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
            default: launch_g<DT, 64, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod); break;
        }
    } else {
        // one row per wave, up to 8 runs of 4 per lane; up to 1024 channels
        // a lane group takes two rows at once, two reductions in flight
        // (62,710 rows x 1024: 83 -> 68 us; four rows measured 74 us)
        if (c <= 1024) launch_g<DT, 64, 4, 2>(s, x, n, c, gamma, beta, eps, silu, y, mod);
        else launch_g<DT, 64, kNormMaxC / 256, 1>(s, x, n, c, gamma, beta, eps, silu, y, mod);
    }
    return hipGetLastError();
}

// ---- GroupNorm over each batch item's rows (SparseGroupNorm32) ----------
// Statistics per (item, group) over the item's rows x the group's channels:
// a partial kernel (one block per (chunk of R rows, item)) writes F64 sums
// and sums of squares per group; a finalize kernel (one wave per (item,
// group)) adds an item's chunks in a fixed lane-strided order and a fixed
// shuffle tree.  R depends only on the shape (gn_chunk_rows), so results
// are deterministic.
constexpr int kGnMaxC = 1024;
constexpr int64_t kGnTargetBlocks = 2048;  // about 8 blocks per CU

// rows per chunk: enough chunks to fill the device, at least 16 rows
__host__ __device__ inline int64_t gn_chunk_rows(int64_t n_batch, int64_t max_rows) {
    int64_t r = (n_batch * max_rows + kGnTargetBlocks - 1) / kGnTargetBlocks;
    r = (r + 15) / 16 * 16;
    return r < 16 ? 16 : (r > 1024 ? 1024 : r);
}

inline int64_t gn_chunks(int64_t n_batch, int64_t max_rows) {
    const int64_t r = gn_chunk_rows(n_batch, max_rows);
    return std::max<int64_t>(1, (max_rows + r - 1) / r);
}

// Lanes take runs of W = 4 * NV channels (16-byte loads for 2-byte types
// with NV = 2); c / W run lanes x floor(256 / (c / W)) row lanes.
template <int DT, int NV>
__global__ __launch_bounds__(256) void gn_partial_kernel(const void* __restrict__ x, int c, int groups,
                                                         const int64_t* __restrict__ off, int rows_per,
                                                         double* __restrict__ part, int chunks) {
    using E = Elem<DT>;
    constexpr int W = 4 * NV;
    constexpr int LS = 256 * W;           // rl_n * c = rl_n * nrun * W <= 256 * W
    __shared__ float ls[2 * LS];          // [row lane][c] sums, then squares
    __shared__ double cs[2 * kGnMaxC];
    const int b = blockIdx.y;
    const int64_t r0 = off[b] + (int64_t)blockIdx.x * rows_per;
    const int64_t r1 = min(off[b + 1], r0 + rows_per);
    const int nrun = c / W;
    const int rl_n = 256 / nrun;          // row lanes
    const int tid = threadIdx.x;
    const int v = tid % nrun, rl = tid / nrun;
    float s[W], q[W];
#pragma unroll
    for (int e = 0; e < W; ++e) s[e] = q[e] = 0.f;
    if (rl < rl_n) {
        int64_t r = r0 + rl;
        // four rows in flight per lane
        for (; r + 3 * rl_n < r1; r += 4 * rl_n) {
            float t[4][W];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int h = 0; h < NV; ++h) E::ld4(x, (r + u * rl_n) * c + W * v + 4 * h, t[u] + 4 * h);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    s[e] += t[u][e];
                    q[e] += t[u][e] * t[u][e];
                }
        }
        for (; r < r1; r += rl_n) {
            float t[W];
#pragma unroll
            for (int h = 0; h < NV; ++h) E::ld4(x, r * c + W * v + 4 * h, t + 4 * h);
#pragma unroll
            for (int e = 0; e < W; ++e) {
                s[e] += t[e];
                q[e] += t[e] * t[e];
            }
        }
#pragma unroll
        for (int e = 0; e < W; ++e) {
            ls[rl * c + W * v + e] = s[e];
            ls[LS + rl * c + W * v + e] = q[e];
        }
    }
    __syncthreads();
    for (int ch = tid; ch < c; ch += 256) {
        double a = 0.0, aa = 0.0;
        for (int k = 0; k < rl_n; ++k) {
            a += ls[k * c + ch];
            aa += ls[LS + k * c + ch];
        }
        cs[ch] = a;
        cs[kGnMaxC + ch] = aa;
    }
    __syncthreads();
    const int cpg = c / groups;
    for (int g = tid; g < groups; g += 256) {
        double a = 0.0, aa = 0.0;
        for (int k = 0; k < cpg; ++k) {
            a += cs[g * cpg + k];
            aa += cs[kGnMaxC + g * cpg + k];
        }
        double* p = part + (((int64_t)b * chunks + blockIdx.x) * groups + g) * 2;
        p[0] = a;
        p[1] = aa;
    }
}

// one 64-lane block per (item, group)
__global__ __launch_bounds__(64) void gn_finalize_kernel(const double* __restrict__ part,
                                                         const int64_t* __restrict__ off, int groups,
                                                         int chunks, int rows_per, int cpg, float eps,
                                                         float* __restrict__ stats) {
    const int i = blockIdx.x;
    const int b = i / groups, g = i % groups;
    const int lane = threadIdx.x;
    const int64_t rows = off[b + 1] - off[b];
    // never past the partials written (callers pass max_rows >= every item's rows)
    const int used = (int)min<int64_t>((rows + rows_per - 1) / rows_per, chunks);
    double a = 0.0, aa = 0.0;
    for (int k = lane; k < used; k += 64) {
        const double* p = part + (((int64_t)b * chunks + k) * groups + g) * 2;
        a += p[0];
        aa += p[1];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        a += __shfl_xor(a, o);
        aa += __shfl_xor(aa, o);
    }
    if (lane == 0) {
        const double cnt = (double)rows * cpg;
        const double mean = cnt > 0 ? a / cnt : 0.0;
        const double var = cnt > 0 ? fmax(aa / cnt - mean * mean, 0.0) : 0.0;
        stats[2 * i] = (float)mean;
        stats[2 * i + 1] = (float)(1.0 / sqrt(var + (double)eps));
    }
}

// y[i] = dt(silu(dt(x[src] * a + b))) with the per-channel coefficients
// a = rstd * gamma, b = beta - a * mean of src's batch item (the fused form
// torch's group_norm evaluates), src = rows[i] (or i); the batch item of src
// by a binary search over the row offsets.  Each lane handles a run of
// 4 * NV channels (16 bytes for 2-byte types with NV = 2).  With TAB the
// block first tabulates a and b for every (item, channel) in LDS
// (n_batch * c <= kGnCoefMax), so a run reads them as two 16-byte words per
// four channels.
constexpr int kGnCoefMax = 4096;

template <int DT, int NV, bool TAB>
__global__ __launch_bounds__(256) void gn_apply_kernel(const void* __restrict__ x, int64_t n_src, int c,
                                                       int groups, const int64_t* __restrict__ off,
                                                       int n_batch, const float* __restrict__ stats,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, int silu,
                                                       const int32_t* __restrict__ rows,
                                                       int64_t n_out, void* __restrict__ y) {
    using E = Elem<DT>;
    constexpr int W = 4 * NV;
    __shared__ __attribute__((aligned(16))) float2 coef[TAB ? kGnCoefMax : 1];
    const int nrun = c / W;
    const int cpg = c / groups;
    auto coef_of = [&](int b, int ch) __attribute__((always_inline)) {
        const int g = ch / cpg;
        const float mean = stats[2 * ((int64_t)b * groups + g)];
        const float rstd = stats[2 * ((int64_t)b * groups + g) + 1];
        const float av = rstd * (gamma ? gamma[ch] : 1.0f);
        return float2{av, (beta ? beta[ch] : 0.0f) - av * mean};
    };
    if constexpr (TAB) {
        for (int k = threadIdx.x; k < n_batch * c; k += blockDim.x) coef[k] = coef_of(k / c, k % c);
        __syncthreads();
    }
    const int64_t total = n_out * nrun;
    const bool small = total < ((int64_t)1 << 32);  // 32-bit row / run split
    for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
         id += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = small ? (int64_t)((uint32_t)id / (uint32_t)nrun) : id / nrun;
        const int c0 = W * (int)(id - i * nrun);
        const int64_t src = rows ? rows[i] : i;
        float o[W];
#pragma unroll
        for (int e = 0; e < W; ++e) o[e] = 0.f;
        if (src >= 0 && src < n_src) {
            int lo = 0, hi = n_batch;  // last b with off[b] <= src
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (off[mid] <= src) lo = mid;
                else hi = mid;
            }
            float t[W];
#pragma unroll
            for (int h = 0; h < NV; ++h) E::ld4(x, src * c + c0 + 4 * h, t + 4 * h);
#pragma unroll
            for (int e = 0; e < W; ++e) {
                float2 ab;
                if constexpr (TAB) ab = coef[lo * c + c0 + e];
                else ab = coef_of(lo, c0 + e);
                float u = t[e] * ab.x + ab.y;
                u = E::round(u);  // GroupNorm32 casts back to the feature dtype
                o[e] = silu ? silu_f32(u) : u;
            }
        }
#pragma unroll
        for (int h = 0; h < NV; ++h) E::st4(y, i * c + c0 + 4 * h, o + 4 * h);
    }
}

template <int DT>
hipError_t launch_gn_stats(hipStream_t s, const void* x, int c, int groups, const int64_t* off,
                           int n_batch, int64_t max_rows, double* part, float eps, float* stats) {
    const int rows_per = (int)gn_chunk_rows(n_batch, max_rows);
    const int chunks = (int)gn_chunks(n_batch, max_rows);
    if (DT != SPC_F32 && c % 8 == 0)
        gn_partial_kernel<DT, 2><<<dim3(chunks, n_batch), 256, 0, s>>>(x, c, groups, off, rows_per,
                                                                       part, chunks);
    else
        gn_partial_kernel<DT, 1><<<dim3(chunks, n_batch), 256, 0, s>>>(x, c, groups, off, rows_per,
                                                                       part, chunks);
    gn_finalize_kernel<<<n_batch * groups, 64, 0, s>>>(part, off, groups, chunks, rows_per,
                                                      c / groups, eps, stats);
    return hipGetLastError();
}

template <int DT>
hipError_t launch_gn_apply(hipStream_t s, const void* x, int64_t n_src, int c, int groups,
                           const int64_t* off, int n_batch, const float* stats, const float* gamma,
                           const float* beta, int silu, const int32_t* rows, int64_t n_out, void* y) {
    const bool wide = DT != SPC_F32 && c % 8 == 0;
    const bool tab = (int64_t)n_batch * c <= kGnCoefMax;
    const int64_t total = n_out * (c / (wide ? 8 : 4));
    // tabulating blocks take more rows each, so the table is built fewer times
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(total, 256), tab ? 4096 : 65536);
#define SPC_GN_APPLY(NV, TAB)                                                                  \
    gn_apply_kernel<DT, NV, TAB><<<grid, 256, 0, s>>>(x, n_src, c, groups, off, n_batch, stats, \
                                                      gamma, beta, silu, rows, n_out, y)
    if (wide && tab) SPC_GN_APPLY(2, true);
    else if (wide) SPC_GN_APPLY(2, false);
    else if (tab) SPC_GN_APPLY(1, true);
    else SPC_GN_APPLY(1, false);
#undef SPC_GN_APPLY
    return hipGetLastError();
}

}  // namespace

}  // namespace spc

using namespace spc;

namespace {

int layernorm_entry(const char* fn, spc_stream_t stream, int dtype, const void* x, int64_t n,
                    int64_t c, const float* gamma, const float* beta, float eps, int silu,
                    void* y, const NormMod& mod) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n < 0 || c <= 0 || c > kNormMaxC || c % 4 != 0 || !(eps >= 0.0f)) {
        set_last_error("%s: unsupported shape n=%lld c=%lld (c a multiple of 4, at most %d) or eps",
                       fn, (long long)n, (long long)c, kNormMaxC);
        return SPC_BAD_SHAPE;
    }
    if (n == 0) return SPC_OK;
    const size_t align = dtype == SPC_F32 ? 16 : 8;
    if (!x || !y || ((uintptr_t)x % align) || ((uintptr_t)y % align) || ((uintptr_t)gamma % 16) ||
        ((uintptr_t)beta % 16)) {
        set_last_error("%s: null or misaligned pointer (gamma / beta 16-byte aligned)", fn);
        return SPC_BAD_ARG;
    }
    hipError_t e;
    if (dtype == SPC_BF16) e = launch_norm<SPC_BF16>(s, x, n, (int)c, gamma, beta, eps, silu, y, mod);
    else if (dtype == SPC_F16) e = launch_norm<SPC_F16>(s, x, n, (int)c, gamma, beta, eps, silu, y, mod);
    else if (dtype == SPC_F32) e = launch_norm<SPC_F32>(s, x, n, (int)c, gamma, beta, eps, silu, y, mod);
    else {
        set_last_error("%s: unknown dtype %d", fn, dtype);
        return SPC_BAD_ARG;
    }
    if (e != hipSuccess) {
        set_last_error("%s: launch failed: %s", fn, hipGetErrorString(e));
        return SPC_HIP_ERROR;
    }
    return SPC_OK;
}

}  // namespace

extern "C" {

int spc_layernorm_silu(spc_stream_t stream, int dtype, const void* x, int64_t n, int64_t c,
                       const float* gamma, const float* beta, float eps, int silu, void* y) {
    return layernorm_entry("spc_layernorm_silu", stream, dtype, x, n, c, gamma, beta, eps, silu,
                           y, NormMod{nullptr, nullptr, nullptr, 0});
}

int spc_layernorm_mod_silu(spc_stream_t stream, int dtype, const void* x, int64_t n, int64_t c,
                           float eps, const float* scale, const float* shift,
                           const int32_t* coords, int64_t n_batch, void* y) {
    if (!scale || !shift || !coords || ((uintptr_t)scale % 16) || ((uintptr_t)shift % 16) ||
        n_batch < 1) {
        set_last_error("spc_layernorm_mod_silu: needs 16-byte aligned scale and shift, coords and "
                       "n_batch >= 1");
        return SPC_BAD_ARG;
    }
    return layernorm_entry("spc_layernorm_mod_silu", stream, dtype, x, n, c, nullptr, nullptr, eps,
                           1, y, NormMod{scale, shift, coords, n_batch});
}

size_t spc_group_norm_workspace_bytes(int64_t n_batch, int64_t max_rows, int64_t groups) {
    if (n_batch <= 0 || max_rows < 0 || groups <= 0) return 0;
    return (size_t)(n_batch * gn_chunks(n_batch, max_rows) * groups * 2 * sizeof(double));
}

int spc_group_norm_stats(spc_stream_t stream, int dtype, const void* x, int64_t c, int64_t groups,
                         const int64_t* offsets, int64_t n_batch, int64_t max_rows, float eps,
                         float* stats, void* workspace, size_t workspace_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (c <= 0 || c > kGnMaxC || c % 4 != 0 || groups <= 0 || c % groups != 0 || n_batch <= 0 ||
        n_batch > 65535 || max_rows < 0 || !(eps >= 0.0f)) {
        set_last_error("spc_group_norm_stats: unsupported shape c=%lld groups=%lld n_batch=%lld "
                       "(c a multiple of 4 and of groups, at most %d)", (long long)c,
                       (long long)groups, (long long)n_batch, kGnMaxC);
        return SPC_BAD_SHAPE;
    }
    if (workspace_bytes < spc_group_norm_workspace_bytes(n_batch, max_rows, groups)) {
        set_last_error("spc_group_norm_stats: workspace too small");
        return SPC_BAD_ARG;
    }
    const size_t align = dtype == SPC_F32 ? 16 : 8;
    if (!x || !offsets || !stats || !workspace || ((uintptr_t)x % align) ||
        ((uintptr_t)workspace % 8)) {
        set_last_error("spc_group_norm_stats: null or misaligned pointer");
        return SPC_BAD_ARG;
    }
    hipError_t e;
    double* part = static_cast<double*>(workspace);
    if (dtype == SPC_BF16) e = launch_gn_stats<SPC_BF16>(s, x, (int)c, (int)groups, offsets, (int)n_batch, max_rows, part, eps, stats);
    else if (dtype == SPC_F16) e = launch_gn_stats<SPC_F16>(s, x, (int)c, (int)groups, offsets, (int)n_batch, max_rows, part, eps, stats);
    else if (dtype == SPC_F32) e = launch_gn_stats<SPC_F32>(s, x, (int)c, (int)groups, offsets, (int)n_batch, max_rows, part, eps, stats);
    else {
        set_last_error("spc_group_norm_stats: unknown dtype %d", dtype);
        return SPC_BAD_ARG;
    }
    if (e != hipSuccess) {
        set_last_error("spc_group_norm_stats: launch failed: %s", hipGetErrorString(e));
        return SPC_HIP_ERROR;
    }
    return SPC_OK;
}

int spc_group_norm_silu(spc_stream_t stream, int dtype, const void* x, int64_t n_src, int64_t c,
                        int64_t groups, const int64_t* offsets, int64_t n_batch, const float* stats,
                        const float* gamma, const float* beta, int silu, const int32_t* rows,
                        int64_t n_out, void* y) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_src < 0 || n_out < 0 || c <= 0 || c > kGnMaxC || c % 4 != 0 || groups <= 0 ||
        c % groups != 0 || n_batch <= 0) {
        set_last_error("spc_group_norm_silu: unsupported shape");
        return SPC_BAD_SHAPE;
    }
    if (n_out == 0) return SPC_OK;
    if (!rows && n_out != n_src) {
        set_last_error("spc_group_norm_silu: rows may be NULL only when n_out == n_src");
        return SPC_BAD_ARG;
    }
    const size_t align = dtype == SPC_F32 ? 16 : 8;
    if (!x || !y || !offsets || !stats || ((uintptr_t)x % align) || ((uintptr_t)y % align) ||
        ((uintptr_t)gamma % 16) || ((uintptr_t)beta % 16)) {
        set_last_error("spc_group_norm_silu: null or misaligned pointer");
        return SPC_BAD_ARG;
    }
    hipError_t e;
    if (dtype == SPC_BF16) e = launch_gn_apply<SPC_BF16>(s, x, n_src, (int)c, (int)groups, offsets, (int)n_batch, stats, gamma, beta, silu, rows, n_out, y);
    else if (dtype == SPC_F16) e = launch_gn_apply<SPC_F16>(s, x, n_src, (int)c, (int)groups, offsets, (int)n_batch, stats, gamma, beta, silu, rows, n_out, y);
    else if (dtype == SPC_F32) e = launch_gn_apply<SPC_F32>(s, x, n_src, (int)c, (int)groups, offsets, (int)n_batch, stats, gamma, beta, silu, rows, n_out, y);
    else {
        set_last_error("spc_group_norm_silu: unknown dtype %d", dtype);
        return SPC_BAD_ARG;
    }
    if (e != hipSuccess) {
        set_last_error("spc_group_norm_silu: launch failed: %s", hipGetErrorString(e));
        return SPC_HIP_ERROR;
    }
    return SPC_OK;
}

}  // extern "C"
