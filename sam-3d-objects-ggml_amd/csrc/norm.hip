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

// G lanes per row, NV runs of 4 per lane (c <= 4 * G * NV), R rows per lane
// group (rows r, r + groups, ...: R independent reductions in flight)
template <int DT, int G, int NV, int R>
__global__ __launch_bounds__(256) void layernorm_silu_kernel(const void* __restrict__ x, int64_t n,
                                                             int c, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             float eps, int silu,
                                                             void* __restrict__ y) {
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
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c0 = 4 * (gl + G * k);
            if (c0 >= c) continue;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float u = v[r][k][e] * rstd;
                if (gamma) u *= gv[k][e];
                if (beta) u += bv[k][e];
                u = E::round(u);  // LayerNorm32 casts back to the feature dtype
                if (silu) u = silu_f32(u);
                o[e] = u;
            }
            E::st4(y, row * c + c0, o);
        }
    }
}

template <int DT, int G, int NV, int R>
void launch_g(hipStream_t s, const void* x, int64_t n, int c, const float* gamma, const float* beta,
              float eps, int silu, void* y) {
    const dim3 grid((unsigned)ceil_div(n, (int64_t)(256 / G) * R));
    layernorm_silu_kernel<DT, G, NV, R><<<grid, dim3(256), 0, s>>>(x, n, c, gamma, beta, eps, silu, y);
}

template <int DT>
hipError_t launch_norm(hipStream_t s, const void* x, int64_t n, int c, const float* gamma,
                       const float* beta, float eps, int silu, void* y) {
    const int runs = c / 4;
    if (runs <= 64) {
        // G = smallest power of two >= runs: several rows per wave
        int g = 1;
        while (g < runs) g <<= 1;
        switch (g) {
            case 1: launch_g<DT, 1, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
            case 2: launch_g<DT, 2, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
            case 4: launch_g<DT, 4, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
            case 8: launch_g<DT, 8, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
            case 16: launch_g<DT, 16, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
            case 32: launch_g<DT, 32, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
            default: launch_g<DT, 64, 1, 1>(s, x, n, c, gamma, beta, eps, silu, y); break;
        }
    } else {
        // one row per wave, up to 8 runs of 4 per lane
        launch_g<DT, 64, kNormMaxC / 256, 1>(s, x, n, c, gamma, beta, eps, silu, y);
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
    if (!x || !y || ((uintptr_t)x % align) || ((uintptr_t)y % align) || ((uintptr_t)gamma % 16) ||
        ((uintptr_t)beta % 16)) {
        set_last_error("spc_layernorm_silu: null or misaligned pointer (gamma / beta 16-byte aligned)");
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
