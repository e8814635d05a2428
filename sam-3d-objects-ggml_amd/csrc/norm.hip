// norm.hip -- row LayerNorm + SiLU over [n, c] features: the prologue of the
// SLAT sparse residual block (structured_latent_flow.py:66-67: norm1 ->
// F.silu; native graph SRC/slat_flow_graph.cpp:331-341).
//
// Each row is handled by G = min(64, c / 4) lanes of a wave (64 / G rows
// per wave), every lane holding runs of 4 consecutive channels (one 8- or
// 16-byte load).  Mean and biased variance are formed in F32 with two
// passes over the registers and group-local shuffles.
#include "common.h"

namespace spc {

namespace {

constexpr int kNormMaxC = 2048;

template <int DT>
struct Elem;
template <>
struct Elem<SPC_F32> {
    __device__ static void ld4(const void* p, int64_t i, float* v) {
        const floatx4 q = *reinterpret_cast<const floatx4*>(static_cast<const float*>(p) + i);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
    __device__ static void st4(void* p, int64_t i, const float* v) {
        *reinterpret_cast<floatx4*>(static_cast<float*>(p) + i) = floatx4{v[0], v[1], v[2], v[3]};
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
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i) =
            u32x2{(uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16),
                  (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16)};
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
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i) =
            u32x2{(uint32_t)f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16),
                  (uint32_t)f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16)};
    }
    __device__ static float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
};

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// G lanes per row, NV runs of 4 per lane (c <= 4 * G * NV)
template <int DT, int G, int NV>
__global__ __launch_bounds__(256) void layernorm_silu_kernel(const void* __restrict__ x, int64_t n,
                                                             int c, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             float eps, int silu,
                                                             void* __restrict__ y) {
    using E = Elem<DT>;
    const int lane = threadIdx.x & 63;
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) / G;
    const int gl = lane % G;  // lane within the row's group
    const bool live = row < n;
    float v[NV][4];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c0 = 4 * (gl + G * k);
        if (live && c0 < c) E::ld4(x, row * c + c0, v[k]);
        else v[k][0] = v[k][1] = v[k][2] = v[k][3] = 0.0f;
        s += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
    }
    const float mean = group_sum<G>(s) / (float)c;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (4 * (gl + G * k) < c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = v[k][e] - mean;
                q += d * d;
            }
        }
    }
    const float rstd = 1.0f / sqrtf(group_sum<G>(q) / (float)c + eps);
    if (!live) return;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c0 = 4 * (gl + G * k);
        if (c0 >= c) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float u = (v[k][e] - mean) * rstd;
            if (gamma) u *= gamma[c0 + e];
            if (beta) u += beta[c0 + e];
            u = E::round(u);  // LayerNorm32 casts back to the feature dtype
            if (silu) u = u / (1.0f + expf(-u));
            o[e] = u;
        }
        E::st4(y, row * c + c0, o);
    }
}

template <int DT>
hipError_t launch_norm(hipStream_t s, const void* x, int64_t n, int c, const float* gamma,
                       const float* beta, float eps, int silu, void* y) {
    const int runs = c / 4;
    const dim3 block(256);
    if (runs <= 64) {
        // G = smallest power of two >= runs: several rows per wave
        int g = 1;
        while (g < runs) g <<= 1;
        const int64_t rows_per_block = 256 / g;
        const dim3 grid((unsigned)ceil_div(n, rows_per_block));
        switch (g) {
            case 1: layernorm_silu_kernel<DT, 1, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
            case 2: layernorm_silu_kernel<DT, 2, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
            case 4: layernorm_silu_kernel<DT, 4, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
            case 8: layernorm_silu_kernel<DT, 8, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
            case 16: layernorm_silu_kernel<DT, 16, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
            case 32: layernorm_silu_kernel<DT, 32, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
            default: layernorm_silu_kernel<DT, 64, 1><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps, silu, y); break;
        }
    } else {
        // one row per wave, up to 8 runs of 4 per lane
        const dim3 grid((unsigned)ceil_div(n, 4));
        layernorm_silu_kernel<DT, 64, kNormMaxC / 256><<<grid, block, 0, s>>>(x, n, c, gamma, beta, eps,
                                                                             silu, y);
    }
    return hipGetLastError();
}

}  // namespace

}  // namespace spc

using namespace spc;

extern "C" {

int spc_layernorm_silu(spc_stream_t stream, int dtype, const void* x, int64_t n, int64_t c,
                       const float* gamma, const float* beta, float eps, int silu, void* y) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n < 0 || c <= 0 || c > kNormMaxC || c % 4 != 0 || !(eps >= 0.0f)) {
        set_last_error("spc_layernorm_silu: unsupported shape n=%lld c=%lld (c a multiple of 4, "
                       "at most %d) or eps", (long long)n, (long long)c, kNormMaxC);
        return SPC_BAD_SHAPE;
    }
    if (n == 0) return SPC_OK;
    const size_t align = dtype == SPC_F32 ? 16 : 8;
    if (!x || !y || ((uintptr_t)x % align) || ((uintptr_t)y % align)) {
        set_last_error("spc_layernorm_silu: null or misaligned pointer");
        return SPC_BAD_ARG;
    }
    hipError_t e;
    if (dtype == SPC_BF16) e = launch_norm<SPC_BF16>(s, x, n, (int)c, gamma, beta, eps, silu, y);
    else if (dtype == SPC_F16) e = launch_norm<SPC_F16>(s, x, n, (int)c, gamma, beta, eps, silu, y);
    else if (dtype == SPC_F32) e = launch_norm<SPC_F32>(s, x, n, (int)c, gamma, beta, eps, silu, y);
    else {
        set_last_error("spc_layernorm_silu: unknown dtype %d", dtype);
        return SPC_BAD_ARG;
    }
    if (e != hipSuccess) {
        set_last_error("spc_layernorm_silu: launch failed: %s", hipGetErrorString(e));
        return SPC_HIP_ERROR;
    }
    return SPC_OK;
}

}  // extern "C"
