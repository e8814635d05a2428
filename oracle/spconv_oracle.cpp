// spconv_oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// CPU restatement of the reference's sparse-voxel convolution path, used as
// the parity checker by tests/, by __graft_entry__.smoke() and as the timed
// CPU baseline ("port") in bench.py.  The product (the HIP library) never
// links, loads or calls this file.
//
// Every function cites the reference source it restates (paths relative to
// the reference repository root):
//   PATCH = cpp_ggml/third_party/ggml-patches/0001-sam3d-ggml-combined.patch
//   SRC   = cpp_ggml/src
//
// Parity pins (what checks each function independently of this file):
//   orc_conv_table_slat / orc_spconv_tables / orc_downsample_map
//       -> compiled reference SlatTables::build (oracle/_ref), golden sha256
//          fixtures, the KAT of SRC/sparse_tables_test.cpp, symmetry and
//          brute-force invariants.
//   orc_conv_table_mesh / orc_subdivide
//       -> compiled reference MeshTables::build (oracle/_ref), the KAT of
//          SRC/mesh_tables_test.cpp, error-code cases.
//   orc_sparse_conv
//       -> closed forms (identity kernel, single-tap shift, linearity) and a
//          dense torch conv3d brute force on small grids (tests/).
//   orc_sparse_conv_blocked
//       -> bit-identical to orc_sparse_conv on random problems of every
//          dtype, layout and tap count (tests/test_oracle_conv.py).
//   orc_stride2_taps
//       -> dense torch conv3d(stride=2) brute force on small grids.
//   orc_scatter_mean
//       -> exact-integer and F16-rounding-history cases whose results are
//          fixed by IEEE binary16 arithmetic (tests/).
//   orc_q8_0_quantize / orc_q8_0_dequant
//       -> hand-computed blocks and the |w - deq| <= d/2 bound.
//       ggml's own quantize_row_q8_0_ref (fp32 reciprocal + roundf) is not
//       in the reference tree: parity against it is unpinned.
//
// Arithmetic: compiled with -ffp-contract=off so every F32 multiply and add
// rounds separately, in the order the reference loops state.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <random>
#include <thread>
#include <tuple>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// IEEE conversions written from the binary16 / bfloat16 definitions
// (round to nearest, ties to even).
// ---------------------------------------------------------------------------
inline uint32_t f32_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline float bits_f32(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    if (e == 0) {
        // zero or subnormal: m * 2^-24 is exact in binary32
        const float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

inline uint16_t f2h(float f) {
    uint32_t u = f32_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
    u &= 0x7fffffffu;
    if (u >= 0x7f800000u) return sign | (u > 0x7f800000u ? 0x7e00 : 0x7c00);
    if (u >= 0x477ff000u) return sign | 0x7c00;  // >= 65520 rounds to inf
    const uint32_t e = u >> 23;
    if (u < 0x38800000u) {  // below 2^-14: binary16 subnormal or zero
        if (e == 0) return sign;  // binary32 subnormals are far below 2^-25
        const uint32_t mant = (u & 0x7fffffu) | 0x800000u;
        const uint32_t s = 126 - e;  // value = mant * 2^-s * 2^-24
        if (s >= 25) return sign;
        uint32_t m = mant >> s;
        const uint32_t rem = mant & ((1u << s) - 1u);
        const uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (m & 1u))) m++;
        return sign | (uint16_t)m;
    }
    uint32_t h = ((e - 127 + 15) << 10) | ((u & 0x7fffffu) >> 13);
    const uint32_t rem = u & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return sign | (uint16_t)h;
}

inline float b2f(uint16_t b) { return bits_f32((uint32_t)b << 16); }

inline uint16_t f2b(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

enum Dtype { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };

inline float load_as_f32(int dtype, const void* p, int64_t i) {
    switch (dtype) {
        case ORC_F16: return h2f(static_cast<const uint16_t*>(p)[i]);
        case ORC_BF16: return b2f(static_cast<const uint16_t*>(p)[i]);
        default: return static_cast<const float*>(p)[i];
    }
}

inline void store_from_f32(int dtype, void* p, int64_t i, float v) {
    switch (dtype) {
        case ORC_F16: static_cast<uint16_t*>(p)[i] = f2h(v); break;
        case ORC_BF16: static_cast<uint16_t*>(p)[i] = f2b(v); break;
        default: static_cast<float*>(p)[i] = v; break;
    }
}

using Key4 = std::tuple<int32_t, int32_t, int32_t, int32_t>;

inline void offset_delta(int o, int32_t& dx, int32_t& dy, int32_t& dz) {
    // SRC/sparse_ops.cpp:108 -- o = kd*9 + kh*3 + kw, centre tap o = 13
    dx = o / 9 - 1;
    dy = (o / 3) % 3 - 1;
    dz = o % 3 - 1;
}

template <typename F>
void run_partitioned(int64_t items, int nthreads, F&& body) {
    // The ggml CPU op's partition: thread ith owns [ith*per, ith*per + per)
    // (PATCH:245-250).
    if (nthreads <= 1) {
        body(0, 1);
        return;
    }
    (void)items;
    std::vector<std::thread> pool;
    for (int ith = 0; ith < nthreads; ++ith) pool.emplace_back(body, ith, nthreads);
    for (auto& t : pool) t.join();
}

struct ConvProblem {
    const void* x;
    const void* w;
    int w_layout;
    int b_dtype;
    const void* bias;
    int y_dtype;
    void* y;
    const int32_t* idx;
    int idx_layout;
    int64_t ntaps, n_out, n_in, channels, out_channels;
};

struct LoadF32 {
    typedef float T;
    static float f(float v) { return v; }
};
struct LoadF16 {
    typedef uint16_t T;
    static float f(uint16_t v) { return h2f(v); }
};
struct LoadBF16 {
    typedef uint16_t T;
    static float f(uint16_t v) { return b2f(v); }
};

// Rows [begin, end) of the F32-accumulate conv.  The element loads are
// resolved at compile time; the arithmetic is the op's: acc = bias, then
// acc += w * x for offsets ascending and channels ascending, each multiply
// and add rounded separately (-ffp-contract=off).
template <typename LX, typename LW>
void conv_rows(const ConvProblem& p, int64_t begin, int64_t end) {
    const auto* x = static_cast<const typename LX::T*>(p.x);
    const auto* w = static_cast<const typename LW::T*>(p.w);
    const int64_t C = p.channels;
    for (int64_t t = begin; t < end; ++t) {
        for (int64_t out = 0; out < p.out_channels; ++out) {
            float acc = p.bias ? load_as_f32(p.b_dtype, p.bias, out) : 0.0f;
            for (int64_t o = 0; o < p.ntaps; ++o) {
                const int32_t s = p.idx_layout == 0 ? p.idx[o * p.n_out + t] : p.idx[t * p.ntaps + o];
                if (s < 0 || s >= p.n_in) continue;
                const int64_t wbase = p.w_layout == 0 ? (out * p.ntaps + o) * C
                                                      : (o * p.out_channels + out) * C;
                const auto* wr = w + wbase;
                const auto* xr = x + (int64_t)s * C;
                for (int64_t c = 0; c < C; ++c) acc += LW::f(wr[c]) * LX::f(xr[c]);
            }
            store_from_f32(p.y_dtype, p.y, t * p.out_channels + out, acc);
        }
    }
}

template <typename LX>
void conv_rows_w(int w_dtype, const ConvProblem& p, int64_t b, int64_t e) {
    switch (w_dtype) {
        case ORC_F16: conv_rows<LX, LoadF16>(p, b, e); break;
        case ORC_BF16: conv_rows<LX, LoadBF16>(p, b, e); break;
        default: conv_rows<LX, LoadF32>(p, b, e); break;
    }
}

void conv_rows_dispatch(int x_dtype, int w_dtype, const ConvProblem& p, int64_t b, int64_t e) {
    switch (x_dtype) {
        case ORC_F16: conv_rows_w<LoadF16>(w_dtype, p, b, e); break;
        case ORC_BF16: conv_rows_w<LoadBF16>(w_dtype, p, b, e); break;
        default: conv_rows_w<LoadF32>(w_dtype, p, b, e); break;
    }
}

// The same conv with the loops reordered for speed: blocks of kRowBlock
// output rows x kOutBlock output channels, weights pre-converted to F32 in
// [tap][cin][cout] order.  Every output element still sees exactly the
// scalar loop's operations in the same order -- acc = bias, then for taps
// ascending (valid ones) and channels ascending acc = acc + w * x, the
// product and the sum each rounded to F32 (-ffp-contract=off keeps them
// separate) -- so the results are bit-identical to conv_rows; only
// independent elements are interleaved, which lets the compiler vectorise
// across output channels.
constexpr int64_t kRowBlock = 32;
constexpr int64_t kOutBlock = 256;

template <typename LX>
void conv_rows_blocked(const ConvProblem& p, const float* wt, int64_t begin, int64_t end) {
    const auto* x = static_cast<const typename LX::T*>(p.x);
    const int64_t C = p.channels, Co = p.out_channels;
    std::vector<float> acc((size_t)(kRowBlock * kOutBlock));
    int64_t rows[kRowBlock];
    const typename LX::T* src[kRowBlock];
    for (int64_t t0 = begin; t0 < end; t0 += kRowBlock) {
        const int64_t rb = std::min(kRowBlock, end - t0);
        for (int64_t o0 = 0; o0 < Co; o0 += kOutBlock) {
            const int64_t ob = std::min(kOutBlock, Co - o0);
            for (int64_t r = 0; r < rb; ++r)
                for (int64_t j = 0; j < ob; ++j)
                    acc[(size_t)(r * kOutBlock + j)] =
                        p.bias ? load_as_f32(p.b_dtype, p.bias, o0 + j) : 0.0f;
            for (int64_t o = 0; o < p.ntaps; ++o) {
                int64_t nv = 0;
                for (int64_t r = 0; r < rb; ++r) {
                    const int64_t t = t0 + r;
                    const int32_t s = p.idx_layout == 0 ? p.idx[o * p.n_out + t] : p.idx[t * p.ntaps + o];
                    if (s < 0 || s >= p.n_in) continue;
                    rows[nv] = r;
                    src[nv] = x + (int64_t)s * C;
                    ++nv;
                }
                if (nv == 0) continue;
                const float* wo = wt + (size_t)(o * C * Co + o0);
                for (int64_t c = 0; c < C; ++c) {
                    const float* __restrict__ wc = wo + (size_t)(c * Co);
                    for (int64_t k = 0; k < nv; ++k) {
                        const float xv = LX::f(src[k][c]);
                        float* __restrict__ a = acc.data() + rows[k] * kOutBlock;
                        for (int64_t j = 0; j < ob; ++j) a[j] = a[j] + wc[j] * xv;
                    }
                }
            }
            for (int64_t r = 0; r < rb; ++r)
                for (int64_t j = 0; j < ob; ++j)
                    store_from_f32(p.y_dtype, p.y, (t0 + r) * Co + o0 + j,
                                   acc[(size_t)(r * kOutBlock + j)]);
        }
    }
}

// Weights as F32 [tap][cin][cout] (exact conversions from any storage dtype).
template <typename LW>
void transpose_weights(const ConvProblem& p, float* wt) {
    const auto* w = static_cast<const typename LW::T*>(p.w);
    const int64_t C = p.channels, Co = p.out_channels;
    for (int64_t co = 0; co < Co; ++co)
        for (int64_t o = 0; o < p.ntaps; ++o) {
            const int64_t wbase = p.w_layout == 0 ? (co * p.ntaps + o) * C : (o * Co + co) * C;
            for (int64_t c = 0; c < C; ++c) wt[(size_t)((o * C + c) * Co + co)] = LW::f(w[wbase + c]);
        }
}

}  // namespace

extern "C" {

// Status codes shared with the HIP library's C ABI.
enum { ORC_OK = 0, ORC_BAD_SHAPE = 1, ORC_BAD_COORD = 2, ORC_DUP_COORD = 3 };

// ---------------------------------------------------------------------------
// a1 (SLAT variant): SlatTables::build's build_conv lambda,
// SRC/sparse_ops.cpp:93-118.  Token-major [n*27]; a missing neighbour is the
// sentinel n.  Duplicate coordinates: std::map::emplace keeps the first row,
// only map owners get their table rows filled, so a later duplicate row keeps
// 27 sentinels (SRC/sparse_ops.cpp:96-100, 105-115).
// ---------------------------------------------------------------------------
int orc_conv_table_slat(const int32_t* coords, int64_t n, int32_t* token_major) {
    if (n <= 0) return ORC_BAD_SHAPE;
    std::map<Key4, int32_t> index;
    for (int64_t i = 0; i < n; ++i)
        index.emplace(Key4{coords[i * 4 + 0], coords[i * 4 + 1], coords[i * 4 + 2],
                           coords[i * 4 + 3]},
                      (int32_t)i);
    std::fill(token_major, token_major + 27 * n, (int32_t)n);
    for (const auto& kv : index) {
        const Key4& k = kv.first;
        const int32_t row = kv.second;
        for (int o = 0; o < 27; ++o) {
            int32_t dx, dy, dz;
            offset_delta(o, dx, dy, dz);
            auto it = index.find(Key4{std::get<0>(k), std::get<1>(k) + dx,
                                      std::get<2>(k) + dy, std::get<3>(k) + dz});
            if (it != index.end()) token_major[(int64_t)row * 27 + o] = it->second;
        }
    }
    return ORC_OK;
}

// ---------------------------------------------------------------------------
// a1 (mesh variant): build_mesh_conv_table, SRC/sparse_ops.cpp:312-346.
// Rejects coordinates outside [0, resolution) and duplicates.
// ---------------------------------------------------------------------------
int orc_conv_table_mesh(const int32_t* coords, int64_t n, int32_t resolution,
                        int32_t* token_major) {
    if (n <= 0) return ORC_BAD_SHAPE;
    std::map<Key4, int32_t> index;
    for (int64_t row = 0; row < n; ++row) {
        const int32_t* c = &coords[row * 4];
        if (c[1] < 0 || c[2] < 0 || c[3] < 0 || c[1] >= resolution || c[2] >= resolution ||
            c[3] >= resolution)
            return ORC_BAD_COORD;
        if (!index.emplace(Key4{c[0], c[1], c[2], c[3]}, (int32_t)row).second)
            return ORC_DUP_COORD;
    }
    std::fill(token_major, token_major + 27 * n, (int32_t)n);
    for (int64_t row = 0; row < n; ++row) {
        const int32_t* c = &coords[row * 4];
        for (int o = 0; o < 27; ++o) {
            int32_t dx, dy, dz;
            offset_delta(o, dx, dy, dz);
            auto it = index.find(Key4{c[0], c[1] + dx, c[2] + dy, c[3] + dz});
            if (it != index.end()) token_major[row * 27 + o] = it->second;
        }
    }
    return ORC_OK;
}

// ---------------------------------------------------------------------------
// a2: build_spconv lambda, SRC/sparse_ops.cpp:120-151.  Offset-major
// [27*n] with -1 for a missing neighbour, one 27-bit mask per token,
// std::stable_sort of tokens by mask, masks permuted into sorted order.
// ---------------------------------------------------------------------------
void orc_spconv_tables(const int32_t* token_major, int64_t n, int32_t* offset_major,
                       int32_t* masks_sorted, int32_t* argsort) {
    std::vector<int32_t> masks((size_t)n, 0);
    std::fill(offset_major, offset_major + 27 * n, -1);
    for (int64_t t = 0; t < n; ++t) {
        argsort[t] = (int32_t)t;
        for (int o = 0; o < 27; ++o) {
            const int32_t row = token_major[t * 27 + o];
            if (row >= 0 && row < n) {
                offset_major[(int64_t)o * n + t] = row;
                masks[(size_t)t] |= (int32_t)(1u << o);
            }
        }
    }
    std::stable_sort(argsort, argsort + n,
                     [&](int32_t a, int32_t b) { return masks[(size_t)a] < masks[(size_t)b]; });
    for (int64_t s = 0; s < n; ++s) masks_sorted[s] = masks[(size_t)argsort[s]];
}

// ---------------------------------------------------------------------------
// a3: the coarse section of SlatTables::build, SRC/sparse_ops.cpp:27-81.
// Coarse key (b, x/2, y/2, z/2) with C truncating division; coarse rows in
// lexicographic key order; children compacted in ascending fine-row order and
// padded with nf; count = |children| + 1 (PyTorch's mean counts the initial
// zero row).  Output buffers are sized for the upper bound nc <= nf.
// Returns nc, or -1 for nf <= 0.
// ---------------------------------------------------------------------------
int64_t orc_downsample_map(const int32_t* coords, int64_t nf, int32_t* fine_to_coarse,
                           int32_t* coarse_coords, int32_t* children, float* counts) {
    if (nf <= 0) return -1;
    std::map<Key4, int32_t> coarse;
    for (int64_t i = 0; i < nf; ++i)
        coarse.emplace(Key4{coords[i * 4 + 0], coords[i * 4 + 1] / 2, coords[i * 4 + 2] / 2,
                            coords[i * 4 + 3] / 2},
                       0);
    int32_t id = 0;
    for (auto& kv : coarse) {
        kv.second = id;
        coarse_coords[(int64_t)id * 4 + 0] = std::get<0>(kv.first);
        coarse_coords[(int64_t)id * 4 + 1] = std::get<1>(kv.first);
        coarse_coords[(int64_t)id * 4 + 2] = std::get<2>(kv.first);
        coarse_coords[(int64_t)id * 4 + 3] = std::get<3>(kv.first);
        ++id;
    }
    const int64_t nc = id;
    std::vector<int32_t> cnt((size_t)nc, 0);
    std::fill(children, children + 8 * nc, (int32_t)nf);
    for (int64_t i = 0; i < nf; ++i) {
        const int32_t c = coarse.at(Key4{coords[i * 4 + 0], coords[i * 4 + 1] / 2,
                                         coords[i * 4 + 2] / 2, coords[i * 4 + 3] / 2});
        fine_to_coarse[i] = c;
        const int slot = cnt[(size_t)c]++;
        if (slot < 8) children[(int64_t)c * 8 + slot] = (int32_t)i;
    }
    // slots are filled in ascending fine-row order, so the reference's
    // compaction pass (SRC/sparse_ops.cpp:73-79) leaves them as they are
    for (int64_t c = 0; c < nc; ++c) counts[c] = (float)(cnt[(size_t)c] + 1);
    return nc;
}

// ---------------------------------------------------------------------------
// Stride-2, kernel-2 tap table (the 64^3 -> 32^3 downsampling conv; the reference runs the
// strided SparseConv3d through spconv, SP/conv/conv_spconv.py:39-50, where
// an input p lands in output p//2 at kernel tap k = p%2 per axis).
// taps[c*8 + k] = fine row at tap k = (x&1)*4 + (y&1)*2 + (z&1) of coarse
// row c, or nf if absent.  Coordinates must be non-negative.
// ---------------------------------------------------------------------------
int orc_stride2_taps(const int32_t* coords, int64_t nf, const int32_t* fine_to_coarse,
                     int64_t nc, int32_t* taps) {
    std::fill(taps, taps + 8 * nc, (int32_t)nf);
    for (int64_t i = 0; i < nf; ++i) {
        const int32_t* c = &coords[i * 4];
        if (c[1] < 0 || c[2] < 0 || c[3] < 0) return ORC_BAD_COORD;
        const int k = (c[1] & 1) * 4 + (c[2] & 1) * 2 + (c[3] & 1);
        int32_t& slot = taps[(int64_t)fine_to_coarse[i] * 8 + k];
        if (slot != (int32_t)nf) return ORC_DUP_COORD;
        slot = (int32_t)i;
    }
    return ORC_OK;
}

// ---------------------------------------------------------------------------
// a4: subdivide_mesh_level, SRC/sparse_ops.cpp:348-371 (child order of
// torch.nonzero(ones(2,2,2)): c = dx*4 + dy*2 + dz, row parent*8 + c).
// keep (optional, [n*8]) prunes children; survivors stay in parent-major
// order and parent[] records each survivor's parent row.  Returns the
// output row count, or -1 for a bad n.
// ---------------------------------------------------------------------------
int64_t orc_subdivide(const int32_t* coords, int64_t n, const uint8_t* keep,
                      int32_t* out_coords, int32_t* parent) {
    if (n <= 0 || n > INT32_MAX / 8) return -1;
    int64_t m = 0;
    for (int64_t p = 0; p < n; ++p) {
        const int32_t* s = &coords[p * 4];
        for (int c = 0; c < 8; ++c) {
            if (keep && !keep[p * 8 + c]) continue;
            out_coords[m * 4 + 0] = s[0];
            out_coords[m * 4 + 1] = s[1] * 2 + c / 4;
            out_coords[m * 4 + 2] = s[2] * 2 + (c / 2) % 2;
            out_coords[m * 4 + 3] = s[3] * 2 + c % 2;
            parent[m] = (int32_t)p;
            ++m;
        }
    }
    return m;
}

// ---------------------------------------------------------------------------
// a5: ggml_compute_forward_sam3d_sparse_conv_f16, PATCH:217-265,
// generalised over storage dtypes and tap count:
//   y[t,co] = round_out( b[co] + sum_{o=0..ntaps-1, s valid} sum_{c} w*x )
// accumulated in F32 in exactly that order (bias first, offsets ascending,
// channels ascending).  Sources outside [0, n_in) are skipped (PATCH:255).
//   idx_layout 0: offset-major [ntaps, n_out] (the op's input, PATCH:254)
//   idx_layout 1: token-major  [n_out, ntaps] (SRC/sparse_ops.cpp:102-116)
//   w_layout   0: [Cout, ntaps, Cin]  (ggml op / spconv KRSC, PATCH:257)
//   w_layout   1: [ntaps, Cout, Cin]  (mesh-decoder GGUF layout,
//                                      convert_sam3d_to_gguf.py:508-511)
// bias may be null (zero).  Threads split output tokens like the op.
// ---------------------------------------------------------------------------
int orc_sparse_conv(int x_dtype, const void* x, int w_dtype, const void* w, int w_layout,
                    int b_dtype, const void* bias, int y_dtype, void* y, const int32_t* idx,
                    int idx_layout, int64_t ntaps, int64_t n_out, int64_t n_in,
                    int64_t channels, int64_t out_channels, int nthreads) {
    if (ntaps <= 0 || n_out < 0 || n_in < 0 || channels <= 0 || out_channels <= 0)
        return ORC_BAD_SHAPE;
    ConvProblem p{x, w, w_layout, b_dtype, bias, y_dtype, y, idx, idx_layout, ntaps, n_out,
                  n_in, channels, out_channels};
    auto body = [&](int ith, int nth) {
        const int64_t per = (n_out + nth - 1) / nth;
        const int64_t begin = std::min(n_out, (int64_t)ith * per);
        const int64_t end = std::min(n_out, begin + per);
        conv_rows_dispatch(x_dtype, w_dtype, p, begin, end);
    };
    run_partitioned(n_out, nthreads, body);
    return ORC_OK;
}

// orc_sparse_conv with blocked, vectorisable loops: same arguments, results
// bit-identical to orc_sparse_conv (see conv_rows_blocked; pinned by
// tests/test_oracle_conv.py), fast enough to check every output row of the
// wide (C = 768 / 1024) convs.
int orc_sparse_conv_blocked(int x_dtype, const void* x, int w_dtype, const void* w, int w_layout,
                            int b_dtype, const void* bias, int y_dtype, void* y,
                            const int32_t* idx, int idx_layout, int64_t ntaps, int64_t n_out,
                            int64_t n_in, int64_t channels, int64_t out_channels, int nthreads) {
    if (ntaps <= 0 || n_out < 0 || n_in < 0 || channels <= 0 || out_channels <= 0)
        return ORC_BAD_SHAPE;
    ConvProblem p{x, w, w_layout, b_dtype, bias, y_dtype, y, idx, idx_layout, ntaps, n_out,
                  n_in, channels, out_channels};
    std::vector<float> wt((size_t)(ntaps * channels * out_channels));
    switch (w_dtype) {
        case ORC_F16: transpose_weights<LoadF16>(p, wt.data()); break;
        case ORC_BF16: transpose_weights<LoadBF16>(p, wt.data()); break;
        default: transpose_weights<LoadF32>(p, wt.data()); break;
    }
    auto body = [&](int ith, int nth) {
        const int64_t per = (n_out + nth - 1) / nth;
        const int64_t begin = std::min(n_out, (int64_t)ith * per);
        const int64_t end = std::min(n_out, begin + per);
        switch (x_dtype) {
            case ORC_F16: conv_rows_blocked<LoadF16>(p, wt.data(), begin, end); break;
            case ORC_BF16: conv_rows_blocked<LoadBF16>(p, wt.data(), begin, end); break;
            default: conv_rows_blocked<LoadF32>(p, wt.data(), begin, end); break;
        }
    };
    run_partitioned(n_out, nthreads, body);
    return ORC_OK;
}

// ---------------------------------------------------------------------------
// Scatter-mean: ggml_compute_forward_sam3d_sparse_scatter_mean,
// PATCH:151-215.  Partial sums kept in the storage dtype (F16 in the
// reference; bf16/f32 follow the same rule), fine rows ascending, rows
// outside [0, nc) skipped, then an F32 division by counts[row].
// Threads own disjoint coarse-row ranges (PATCH:185-190).
// ---------------------------------------------------------------------------
int orc_scatter_mean(int dtype, const void* features, const int32_t* rows, const float* counts,
                     void* out, int64_t channels, int64_t nf, int64_t nc, int nthreads) {
    if (channels <= 0 || nf < 0 || nc < 0) return ORC_BAD_SHAPE;
    auto body = [&](int ith, int nth) {
        const int64_t per = (nc + nth - 1) / nth;
        const int64_t begin = std::min(nc, (int64_t)ith * per);
        const int64_t end = std::min(nc, begin + per);
        for (int64_t r = begin; r < end; ++r)
            for (int64_t c = 0; c < channels; ++c) store_from_f32(dtype, out, r * channels + c, 0.0f);
        for (int64_t i = 0; i < nf; ++i) {
            const int32_t r = rows[i];
            if (r < begin || r >= end) continue;
            for (int64_t c = 0; c < channels; ++c) {
                const int64_t di = (int64_t)r * channels + c;
                store_from_f32(dtype, out, di,
                               load_as_f32(dtype, out, di) +
                                   load_as_f32(dtype, features, i * channels + c));
            }
        }
        for (int64_t r = begin; r < end; ++r)
            for (int64_t c = 0; c < channels; ++c) {
                const int64_t di = r * channels + c;
                store_from_f32(dtype, out, di, load_as_f32(dtype, out, di) / counts[r]);
            }
    };
    run_partitioned(nc, nthreads, body);
    return ORC_OK;
}

// ---------------------------------------------------------------------------
// a10: quantize_q8_0, cpp_ggml/scripts/gguf_schema.py:14-24.
// Per block of 32: amax = max|w| (F32; 0 -> 1e-12); d = fp16(amax / 127)
// (F32 division, then round to binary16); q = clip(rint(w / f32(d)),
// -127, 127) with rint = round half to even.  Block = [fp16 d][int8 q[32]],
// 34 bytes.  When d rounds to zero, numpy's w/0 gives +-inf (clipped to
// +-127) and 0/0 gives NaN, whose int8 cast yields 0 on x86; that outcome
// is reproduced.
// ---------------------------------------------------------------------------
int orc_q8_0_quantize(const float* w, int64_t n, uint8_t* out) {
    if (n < 0 || n % 32 != 0) return ORC_BAD_SHAPE;
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* wb = w + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(wb[j]));
        if (amax == 0.0f) amax = 1e-12f;
        const uint16_t dh = f2h(amax / 127.0f);
        const float d = h2f(dh);
        uint8_t* ob = out + b * 34;
        std::memcpy(ob, &dh, 2);
        for (int j = 0; j < 32; ++j) {
            int q;
            if (d == 0.0f) {
                q = wb[j] > 0.0f ? 127 : (wb[j] < 0.0f ? -127 : 0);
            } else {
                float v = std::nearbyint(wb[j] / d);  // default mode: ties to even
                v = std::min(127.0f, std::max(-127.0f, v));
                q = (int)v;
            }
            ob[2 + j] = (uint8_t)(int8_t)q;
        }
    }
    return ORC_OK;
}

// Dequantize Q8_0 blocks: y = f32(d) * q (exact in F32), then stored in
// out_dtype.  The reference feeds f16(f32(d)*q) to its GEMM
// (SRC/slat_flow_graph.cpp:24-27 via ggml_cast).
int orc_q8_0_dequant(const uint8_t* blocks, int64_t nblocks, int out_dtype, void* out) {
    for (int64_t b = 0; b < nblocks; ++b) {
        uint16_t dh;
        std::memcpy(&dh, blocks + b * 34, 2);
        const float d = h2f(dh);
        for (int j = 0; j < 32; ++j) {
            const int8_t q = (int8_t)blocks[b * 34 + 2 + j];
            store_from_f32(out_dtype, out, b * 32 + j, d * (float)q);
        }
    }
    return ORC_OK;
}

// Inputs of one case of the reference's scatter-mean regression test
// (SRC/scatter_mean_backend_test.cpp:35-75), drawn with the same engine and
// distributions in the same order: f16 features uniform in [-4, 4); the
// first min(nc, nf) fine rows hit coarse rows 0.. in order; every later row
// draws rng() % 16 -- 15 -> -1, 14 -> nc (both skipped), else a uniform
// coarse row; counts = hits per coarse row.
void orc_scatter_case(int64_t channels, int64_t nf, int64_t nc, int32_t seed,
                      uint16_t* features, int32_t* rows, float* counts) {
    std::mt19937 rng((uint32_t)seed);
    std::uniform_real_distribution<float> uniform(-4.0f, 4.0f);
    for (int64_t i = 0; i < channels * nf; ++i) features[i] = f2h(uniform(rng));
    std::uniform_int_distribution<int32_t> pick(0, (int32_t)nc - 1);
    const int64_t pinned = std::min(nc, nf);
    for (int64_t i = 0; i < pinned; ++i) rows[i] = (int32_t)i;
    for (int64_t i = pinned; i < nf; ++i) {
        const uint32_t draw = rng() % 16;
        if (draw == 15) rows[i] = -1;
        else if (draw == 14) rows[i] = (int32_t)nc;
        else rows[i] = pick(rng);
    }
    for (int64_t r = 0; r < nc; ++r) counts[r] = 0.0f;
    for (int64_t i = 0; i < nf; ++i)
        if (rows[i] >= 0 && rows[i] < nc) counts[rows[i]] += 1.0f;
}

// Scalar conversions exposed for tests.
void orc_f32_to_f16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f2h(in[i]);
}
void orc_f16_to_f32(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = h2f(in[i]);
}
void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = f2b(in[i]);
}

}  // extern "C"
