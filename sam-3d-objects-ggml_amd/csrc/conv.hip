// conv.hip -- C ABI of the sparse convolution (kernel in conv_kernel.h):
// argument checks, dispatch by dtype, the MFMA-fragment weight packer, the
// Q8_0 block repacker and the reference-compatible spconv bridge.
#include "conv_kernel.h"

namespace spc {

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename T, bool Q8>
size_t packed_quant_bytes(int64_t ntaps, int64_t cin, int64_t cout) {
    return (size_t)ntaps * cin * cout * Panel<T, Q8>::WB;
}

// One thread per 16-byte panel word: panel (tap, chunk, c32), word g, lane.
template <typename T, bool Q8>
__global__ void pack_weights_kernel(const uint8_t* __restrict__ w, u32x4* __restrict__ out,
                                    int ntaps, int cin, int cout) {
    using P = Panel<T, Q8>;
    const int kch = cin / P::KC;
    const int ncol32 = cout / 32;
    const int64_t words = (int64_t)ntaps * kch * ncol32 * P::NG * 64;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= words) return;
    const int lane = (int)(id % 64);
    const int64_t rest = id / 64;
    const int g = (int)(rest % P::NG);
    const int64_t panel = rest / P::NG;
    const int c32 = (int)(panel % ncol32);
    const int64_t tk = panel / ncol32;
    const int kc = (int)(tk % kch);
    const int o = (int)(tk / kch);
    const int co = c32 * 32 + (lane & 31);
    uint8_t bytes[16];
    constexpr int BPK = 16 / P::G;  // bytes per k-step
#pragma unroll
    for (int i = 0; i < P::G; ++i) {
        const int ks = g * P::G + i;
        const int64_t el = ((int64_t)co * ntaps + o) * cin + (int64_t)kc * P::KC +
                           ks * P::KSUB + (lane >> 5) * P::EPL;
#pragma unroll
        for (int b = 0; b < BPK; ++b) bytes[i * BPK + b] = w[el * P::WB + b];
    }
    uint32_t v[4];
#pragma unroll
    for (int h = 0; h < 4; ++h)
        v[h] = (uint32_t)bytes[4 * h] | ((uint32_t)bytes[4 * h + 1] << 8) |
               ((uint32_t)bytes[4 * h + 2] << 16) | ((uint32_t)bytes[4 * h + 3] << 24);
    out[id] = u32x4{v[0], v[1], v[2], v[3]};
}

// Q8_0 scales as f32 per (tap, chunk, co): a 32-channel chunk is one block.
__global__ void pack_scales_kernel(const uint16_t* __restrict__ d, float* __restrict__ out,
                                   int ntaps, int cin, int cout) {
    const int kch = cin / 32;
    const int64_t n = (int64_t)ntaps * kch * cout;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n) return;
    const int co = (int)(id % cout);
    const int64_t tk = id / cout;
    const int kc = (int)(tk % kch);
    const int o = (int)(tk / kch);
    out[id] = f16_bits_to_f32(d[(((int64_t)co * ntaps + o) * cin + (int64_t)kc * 32) >> 5]);
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

int check_shape(const char* fn, int64_t ntaps, int64_t cin, int64_t cout) {
    if ((ntaps != 27 && ntaps != 8) || cin <= 0 || cout <= 0 || cin % 32 != 0 ||
        cout % 32 != 0 || cin > (1 << 16) || cout > (1 << 16)) {
        set_last_error("%s: unsupported shape ntaps=%lld cin=%lld cout=%lld (ntaps 27 or 8, "
                       "cin and cout multiples of 32)",
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

int spc_conv_pack_weights(spc_stream_t stream, int w_dtype, const void* w, const void* w_scale,
                          int64_t ntaps, int64_t cin, int64_t cout, void* packed) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = check_shape("spc_conv_pack_weights", ntaps, cin, cout);
    if (st != SPC_OK) return st;
    if (!w || !packed || !aligned16(packed) || (w_dtype == SPC_Q8_0 && !w_scale)) {
        set_last_error("spc_conv_pack_weights: null / misaligned pointer");
        return SPC_BAD_ARG;
    }
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    u32x4* out = static_cast<u32x4*>(packed);
    switch (w_dtype) {
        case SPC_F32: {
            const int64_t words = (int64_t)packed_quant_bytes<float, false>(ntaps, cin, cout) / 16;
            pack_weights_kernel<float, false><<<(unsigned)ceil_div(words, 256), 256, 0, s>>>(
                wb, out, (int)ntaps, (int)cin, (int)cout);
            break;
        }
        case SPC_F16:
        case SPC_BF16: {
            const int64_t words = (int64_t)packed_quant_bytes<__bf16, false>(ntaps, cin, cout) / 16;
            pack_weights_kernel<__bf16, false><<<(unsigned)ceil_div(words, 256), 256, 0, s>>>(
                wb, out, (int)ntaps, (int)cin, (int)cout);
            break;
        }
        case SPC_Q8_0: {
            const size_t qbytes = packed_quant_bytes<__bf16, true>(ntaps, cin, cout);
            const int64_t words = (int64_t)qbytes / 16;
            pack_weights_kernel<__bf16, true><<<(unsigned)ceil_div(words, 256), 256, 0, s>>>(
                wb, out, (int)ntaps, (int)cin, (int)cout);
            float* sc = reinterpret_cast<float*>(static_cast<char*>(packed) + align_up(qbytes, 256));
            const int64_t ns = ntaps * (cin / 32) * cout;
            pack_scales_kernel<<<(unsigned)ceil_div(ns, 256), 256, 0, s>>>(
                static_cast<const uint16_t*>(w_scale), sc, (int)ntaps, (int)cin, (int)cout);
            break;
        }
        default:
            set_last_error("spc_conv_pack_weights: unknown dtype %d", w_dtype);
            return SPC_BAD_ARG;
    }
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_sparse_conv(spc_stream_t stream, int dtype, const void* x, int w_dtype, int w_layout,
                    const void* w, const void* w_scale, const void* bias, void* y,
                    const int32_t* idx, int idx_layout, const int32_t* row_perm, int64_t ntaps,
                    int64_t n_out, int64_t n_in, int64_t cin, int64_t cout) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = check_shape("spc_sparse_conv", ntaps, cin, cout);
    if (st != SPC_OK) return st;
    if (n_out < 0 || n_in < 0 || n_out > INT32_MAX || n_in > INT32_MAX) {
        set_last_error("spc_sparse_conv: n_out=%lld n_in=%lld out of range", (long long)n_out,
                       (long long)n_in);
        return SPC_BAD_SHAPE;
    }
    if (n_out == 0) return SPC_OK;
    if (!x || !w || !y || !idx || !aligned16(x) || !aligned16(w) ||
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

void sam3d_spconv_f16_forward(spc_stream_t stream, const void* input, const void* weight,
                              const void* bias, void* output, const int32_t* indices,
                              const uint32_t* mask, const int32_t* mask_argsort, int64_t tokens,
                              int64_t channels, int64_t output_channels) {
    (void)mask;  // each tile's tap set is formed from the indices themselves
    spc_sparse_conv(stream, SPC_F16, input, SPC_F16, SPC_W_KRSC, weight, nullptr, bias, output,
                    indices, SPC_IDX_OFFSET_MAJOR, mask_argsort, 27, tokens, tokens, channels,
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
