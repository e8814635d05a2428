// conv.hip -- sparse convolution as gather -> implicit GEMM -> store on
// CDNA4 matrix cores (gfx950).
//
// Arithmetic contract: the ggml CPU op ggml_compute_forward_sam3d_sparse_
// conv_f16 (PATCH:217-265): y[t,co] = bias[co] + sum over valid taps o and
// channels c of w[co,o,c] * x[idx(t,o),c], accumulated in F32 and rounded
// once to the output dtype.  Taps whose source is outside [0, n_in) add
// nothing (PATCH:255).
//
// Kernel structure (output-stationary implicit GEMM):
//   * a workgroup owns a TM x TN output tile (TM rows in processing order,
//     TN output channels); 4 waves split it WM x WN; each wave accumulates
//     (TM/WM) x (TN/WN) with 32x32 MFMA tiles in F32.
//   * at start the tile's ntaps x TM neighbour indices go to LDS and the OR
//     of the rows' valid-tap bits is formed; taps no row of the tile uses
//     are skipped entirely (the per-tile offset set of the reference's
//     spconv kernel, cpp_ggml/third_party/sam3d-spconv/src/.../
//     ConvKernel_conv_kernel.cu:62-80).
//   * K loop over (active tap, KC-channel chunk): the gathered A tile
//     (TM rows x KC channels, zero rows for missing taps) and the weight
//     tile (TN x KC) are staged in LDS with 16-byte loads (each row chunk is
//     a contiguous 128-byte (KC=64 bf16) segment of a feature row), rows
//     padded by 16 bytes against bank conflicts; the next stage's global
//     loads are issued before the current stage's MFMAs (register
//     prefetch).
//   * Q8_0: int8 quants + fp16 block scales are dequantised in registers
//     on their way into LDS: w = bf16(f32(d) * q).
//   * epilogue: + bias in F32, one rounding, direct store of each output
//     row (each output element written exactly once, no atomics).
//   * tiles are mapped XCD-major: workgroup b runs on XCD b % 8, and each
//     XCD receives a contiguous range of row tiles (all N tiles of a row
//     tile together), so a neighbourhood's gathered feature rows stay in
//     that XCD's L2.
#include "common.h"

namespace spc {

namespace {

template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
    static constexpr int KSUB = 16;  // K per instruction
    static constexpr int EPL = 8;    // elements per lane per operand
    typedef bf16x8 frag;
    __device__ static floatx16 mma(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static uint16_t cvt(float v) { return f32_to_bf16_bits(v); }
    __device__ static float ld(const void* p, int64_t i) {
        return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
};

template <>
struct Mfma<_Float16> {
    static constexpr int KSUB = 16;
    static constexpr int EPL = 8;
    typedef f16x8 frag;
    __device__ static floatx16 mma(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    __device__ static uint16_t cvt(float v) { return f32_to_f16_bits(v); }
    __device__ static float ld(const void* p, int64_t i) {
        return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
};

template <>
struct Mfma<float> {
    static constexpr int KSUB = 2;
    static constexpr int EPL = 1;
    typedef float frag;
    __device__ static floatx16 mma(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __device__ static float cvt(float v) { return v; }
    __device__ static float ld(const void* p, int64_t i) {
        return static_cast<const float*>(p)[i];
    }
};

struct ConvArgs {
    const void* x;
    const void* w;
    const uint16_t* wscale;
    const void* bias;
    void* y;
    const int32_t* idx;
    const int32_t* row_perm;
    int64_t n_out;
    int64_t n_in;
    int32_t idx_layout;
    int32_t ntaps;
    int32_t cin;
    int32_t cout;
    int32_t tiles_n;
    int64_t total_tiles;
    int64_t tiles_per_xcd;
};

constexpr int kMaxTaps = 27;

template <typename T, bool Q8, int TM, int TN, int KC, int WM, int WN>
__global__ __launch_bounds__(256) void conv_kernel(ConvArgs a) {
    using M = Mfma<T>;
    constexpr int ES = sizeof(T);
    constexpr int CH = 16 / ES;        // elements per 16-byte chunk
    constexpr int CPR = KC / CH;       // chunks per staged row
    constexpr int PITCH = KC + CH;     // LDS row pitch (elements), +16 bytes
    constexpr int A_CHUNKS = TM * CPR;
    constexpr int B_CHUNKS = TN * CPR;
    constexpr int A_PER_T = (A_CHUNKS + 255) / 256;
    constexpr int B_PER_T = (B_CHUNKS + 255) / 256;
    constexpr int WTM = TM / WM;
    constexpr int WTN = TN / WN;
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    static_assert(A_CHUNKS % 256 == 0 || A_CHUNKS < 256, "staging geometry");
    static_assert(B_CHUNKS % 256 == 0 || B_CHUNKS < 256, "staging geometry");
    static_assert(WM * WN == 4 && FM >= 1 && FN >= 1, "wave geometry");
    static_assert(!Q8 || ES == 2, "Q8_0 weights feed 16-bit MFMA operands");

    __shared__ __attribute__((aligned(16))) T As[TM * PITCH];
    __shared__ __attribute__((aligned(16))) T Bs[TN * PITCH];
    __shared__ int32_t sidx[kMaxTaps * TM];  // [tap][row]
    __shared__ int32_t srow[TM];
    __shared__ uint32_t smask;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // XCD-major tile mapping
    const int64_t xcd = blockIdx.x & 7;
    const int64_t local = blockIdx.x >> 3;
    const int64_t tile = xcd * a.tiles_per_xcd + local;
    if (local >= a.tiles_per_xcd || tile >= a.total_tiles) return;
    const int64_t tm = tile / a.tiles_n;
    const int tn = (int)(tile % a.tiles_n);
    const int64_t r0 = tm * TM;
    const int co0 = tn * TN;
    const int ntaps = a.ntaps;

    if (tid == 0) smask = 0;
    for (int r = tid; r < TM; r += 256) {
        const int64_t rr = r0 + r;
        int32_t t = -1;
        if (rr < a.n_out) t = a.row_perm ? a.row_perm[rr] : (int32_t)rr;
        if (t >= a.n_out) t = -1;  // a bad permutation entry writes nothing
        srow[r] = t;
    }
    __syncthreads();
    uint32_t my_mask = 0;
    for (int e = tid; e < TM * ntaps; e += 256) {
        int r, o;
        if (a.idx_layout == SPC_IDX_TOKEN_MAJOR) {
            r = e / ntaps;
            o = e % ntaps;
        } else {
            o = e / TM;
            r = e % TM;
        }
        const int32_t t = srow[r];
        int32_t src = -1;
        if (t >= 0) {
            src = a.idx_layout == SPC_IDX_TOKEN_MAJOR ? a.idx[(int64_t)t * ntaps + o]
                                                      : a.idx[(int64_t)o * a.n_out + t];
            if (src < 0 || src >= a.n_in) src = -1;
        }
        sidx[o * TM + r] = src;
        if (src >= 0) my_mask |= 1u << o;
    }
    // wave OR-reduce, then one LDS atomic per wave
    for (int off = 32; off > 0; off >>= 1) my_mask |= __shfl_xor(my_mask, off);
    if (lane == 0 && my_mask) atomicOr(&smask, my_mask);
    __syncthreads();
    const uint32_t tile_mask = smask;
    const int kchunks = a.cin / KC;
    const int nsteps = __popc(tile_mask) * kchunks;

    const int wm = wave / WN;
    const int wn = wave % WN;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[i][j][k] = 0.0f;

    const char* xb = static_cast<const char*>(a.x);
    const char* wb = static_cast<const char*>(a.w);

    uint4 ra[A_PER_T];
    uint4 rb[B_PER_T];
    float rs[Q8 ? B_PER_T : 1];

    // prefetch cursor (tap, chunk) -- uniform across the workgroup
    uint32_t pf_mask = tile_mask;
    int pf_o = pf_mask ? __ffs(pf_mask) - 1 : 0;
    int pf_kc = 0;

    auto load_stage = [&]() {
        const int o = pf_o;
        const int kc = pf_kc;
#pragma unroll
        for (int j = 0; j < A_PER_T; ++j) {
            const int ch = tid + j * 256;
            if (A_CHUNKS < 256 && ch >= A_CHUNKS) break;
            const int r = ch / CPR;
            const int seg = ch % CPR;
            const int32_t src = sidx[o * TM + r];
            if (src >= 0) {
                ra[j] = *reinterpret_cast<const uint4*>(
                    xb + ((int64_t)src * a.cin + (int64_t)kc * KC + seg * CH) * ES);
            } else {
                ra[j] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < B_PER_T; ++j) {
            const int ch = tid + j * 256;
            if (B_CHUNKS < 256 && ch >= B_CHUNKS) break;
            const int n = ch / CPR;
            const int seg = ch % CPR;
            const int64_t welem =
                ((int64_t)(co0 + n) * ntaps + o) * a.cin + (int64_t)kc * KC + seg * CH;
            if (Q8) {
                const uint2 q = *reinterpret_cast<const uint2*>(wb + welem);
                rb[j] = make_uint4(q.x, q.y, 0, 0);
                rs[j] = f16_bits_to_f32(a.wscale[welem >> 5]);
            } else {
                rb[j] = *reinterpret_cast<const uint4*>(wb + welem * ES);
            }
        }
        // advance the cursor
        if (++pf_kc == kchunks) {
            pf_kc = 0;
            pf_mask &= pf_mask - 1;
            pf_o = pf_mask ? __ffs(pf_mask) - 1 : 0;
        }
    };

    auto store_stage = [&]() {
#pragma unroll
        for (int j = 0; j < A_PER_T; ++j) {
            const int ch = tid + j * 256;
            if (A_CHUNKS < 256 && ch >= A_CHUNKS) break;
            const int r = ch / CPR;
            const int seg = ch % CPR;
            *reinterpret_cast<uint4*>(&As[r * PITCH + seg * CH]) = ra[j];
        }
#pragma unroll
        for (int j = 0; j < B_PER_T; ++j) {
            const int ch = tid + j * 256;
            if (B_CHUNKS < 256 && ch >= B_CHUNKS) break;
            const int n = ch / CPR;
            const int seg = ch % CPR;
            if (Q8) {
                const uint32_t qw[2] = {rb[j].x, rb[j].y};
                uint32_t packed[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t word = qw[h >> 1];
                    const int sh = (h & 1) * 16;
                    const int8_t q0 = (int8_t)((word >> sh) & 0xff);
                    const int8_t q1 = (int8_t)((word >> (sh + 8)) & 0xff);
                    const uint16_t b0 = f32_to_bf16_bits(rs[j] * (float)q0);
                    const uint16_t b1 = f32_to_bf16_bits(rs[j] * (float)q1);
                    packed[h] = (uint32_t)b0 | ((uint32_t)b1 << 16);
                }
                *reinterpret_cast<uint4*>(&Bs[n * PITCH + seg * CH]) =
                    make_uint4(packed[0], packed[1], packed[2], packed[3]);
            } else {
                *reinterpret_cast<uint4*>(&Bs[n * PITCH + seg * CH]) = rb[j];
            }
        }
    };

    if (nsteps > 0) load_stage();
    for (int step = 0; step < nsteps; ++step) {
        __syncthreads();
        store_stage();
        __syncthreads();
        if (step + 1 < nsteps) load_stage();
#pragma unroll
        for (int ks = 0; ks < KC / M::KSUB; ++ks) {
            typename M::frag af[FM];
            typename M::frag bf[FN];
            const int kof = ks * M::KSUB + (lane >> 5) * M::EPL;
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const typename M::frag*>(
                    &As[(wm * WTM + i * 32 + (lane & 31)) * PITCH + kof]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const typename M::frag*>(
                    &Bs[(wn * WTN + j * 32 + (lane & 31)) * PITCH + kof]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = M::mma(af[i], bf[j], acc[i][j]);
        }
    }

    // epilogue: 32x32 accumulator layout -- element k of lane l holds
    // row 8*(k/4) + 4*(l/32) + k%4, column l%32
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = co0 + wn * WTN + j * 32 + (lane & 31);
        const float bv = a.bias ? M::ld(a.bias, col) : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int rl = wm * WTM + i * 32 + 8 * (k >> 2) + 4 * (lane >> 5) + (k & 3);
                const int32_t t = srow[rl];
                if (t >= 0) {
                    const float v = acc[i][j][k] + bv;
                    if constexpr (ES == 4) {
                        static_cast<float*>(a.y)[(int64_t)t * a.cout + col] = v;
                    } else {
                        static_cast<uint16_t*>(a.y)[(int64_t)t * a.cout + col] = M::cvt(v);
                    }
                }
            }
        }
    }
}

template <typename T, bool Q8, int TM, int TN, int KC, int WM, int WN>
hipError_t launch(hipStream_t s, ConvArgs a) {
    const int64_t tiles_m = ceil_div(a.n_out, TM);
    a.tiles_n = a.cout / TN;
    a.total_tiles = tiles_m * a.tiles_n;
    a.tiles_per_xcd = ceil_div(a.total_tiles, 8);
    const int64_t grid = a.tiles_per_xcd * 8;
    if (grid == 0) return hipSuccess;
    conv_kernel<T, Q8, TM, TN, KC, WM, WN><<<(unsigned)grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

// Tile selection: TN = largest of {128, 64, 32} dividing cout; KC = 128-byte
// rows (64 x 16-bit or 32 x f32) when cin allows, else 64-byte rows.
template <typename T, bool Q8>
hipError_t dispatch(hipStream_t s, const ConvArgs& a) {
    constexpr int KC_BIG = 128 / sizeof(T);
    constexpr int KC_SMALL = 64 / sizeof(T);
    const bool big = a.cin % KC_BIG == 0;
    if (a.cout % 128 == 0)
        return big ? launch<T, Q8, 128, 128, KC_BIG, 2, 2>(s, a)
                   : launch<T, Q8, 128, 128, KC_SMALL, 2, 2>(s, a);
    if (a.cout % 64 == 0)
        return big ? launch<T, Q8, 128, 64, KC_BIG, 4, 1>(s, a)
                   : launch<T, Q8, 128, 64, KC_SMALL, 4, 1>(s, a);
    return big ? launch<T, Q8, 128, 32, KC_BIG, 4, 1>(s, a)
               : launch<T, Q8, 128, 32, KC_SMALL, 4, 1>(s, a);
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
    uint4* dst = reinterpret_cast<uint4*>(qs + b * 32);
    dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
    dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace spc

using namespace spc;

extern "C" {

int spc_sparse_conv(spc_stream_t stream, int dtype, const void* x, int w_dtype, const void* w,
                    const void* w_scale, const void* bias, void* y, const int32_t* idx,
                    int idx_layout, const int32_t* row_perm, int64_t ntaps, int64_t n_out,
                    int64_t n_in, int64_t cin, int64_t cout) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_out < 0 || n_in < 0 || ntaps <= 0 || ntaps > kMaxTaps || cin <= 0 || cout <= 0 ||
        cin % 32 != 0 || cout % 32 != 0 || n_out > INT32_MAX || n_in > INT32_MAX) {
        set_last_error("spc_sparse_conv: unsupported shape ntaps=%lld n_out=%lld n_in=%lld "
                       "cin=%lld cout=%lld (needs ntaps<=27, cin%%32==0, cout%%32==0)",
                       (long long)ntaps, (long long)n_out, (long long)n_in, (long long)cin,
                       (long long)cout);
        return SPC_BAD_SHAPE;
    }
    if (n_out == 0) return SPC_OK;
    if (!x || !w || !y || !idx || !aligned16(x) || !aligned16(w) ||
        (idx_layout != SPC_IDX_TOKEN_MAJOR && idx_layout != SPC_IDX_OFFSET_MAJOR)) {
        set_last_error("spc_sparse_conv: null / misaligned pointer or bad idx_layout");
        return SPC_BAD_ARG;
    }
    ConvArgs a{};
    a.x = x;
    a.w = w;
    a.wscale = static_cast<const uint16_t*>(w_scale);
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
    hipError_t e = hipSuccess;
    if (w_dtype == SPC_Q8_0) {
        if (dtype != SPC_BF16 || !w_scale) {
            set_last_error("spc_sparse_conv: Q8_0 weights need bf16 activations and w_scale");
            return SPC_BAD_ARG;
        }
        e = dispatch<__bf16, true>(s, a);
    } else if (w_dtype != dtype) {
        set_last_error("spc_sparse_conv: w_dtype %d must equal dtype %d", w_dtype, dtype);
        return SPC_BAD_ARG;
    } else if (dtype == SPC_BF16) {
        e = dispatch<__bf16, false>(s, a);
    } else if (dtype == SPC_F16) {
        e = dispatch<_Float16, false>(s, a);
    } else if (dtype == SPC_F32) {
        e = dispatch<float, false>(s, a);
    } else {
        set_last_error("spc_sparse_conv: unknown dtype %d", dtype);
        return SPC_BAD_ARG;
    }
    if (e != hipSuccess) return hip_status(e, "conv_kernel launch");
    return SPC_OK;
}

void sam3d_spconv_f16_forward(spc_stream_t stream, const void* input, const void* weight,
                              const void* bias, void* output, const int32_t* indices,
                              const uint32_t* mask, const int32_t* mask_argsort, int64_t tokens,
                              int64_t channels, int64_t output_channels) {
    (void)mask;  // the kernel forms each tile's tap set from the indices
    spc_sparse_conv(stream, SPC_F16, input, SPC_F16, weight, nullptr, bias, output, indices,
                    SPC_IDX_OFFSET_MAJOR, mask_argsort, 27, tokens, tokens, channels,
                    output_channels);
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

}  // extern "C"
