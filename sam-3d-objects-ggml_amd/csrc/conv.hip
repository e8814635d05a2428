// conv.hip -- sparse convolution as gather -> implicit GEMM -> store on
// CDNA4 matrix cores (gfx950).
//
// Arithmetic contract: the ggml CPU op ggml_compute_forward_sam3d_sparse_
// conv_f16 (PATCH:217-265): y[t,co] = bias[co] + sum over valid taps o and
// channels c of w[co,o,c] * x[idx(t,o),c], accumulated in F32 and rounded
// once to the output dtype.  Taps whose source is outside [0, n_in) add
// nothing (PATCH:255).
//
// Kernel structure (output-stationary implicit GEMM over a deduplicated gather):
//   * a workgroup (8 waves) owns a 256-row x TN output tile (rows in processing order,
//     natural = lexicographic by default); 4 waves split it WM x WN and
//     accumulate 32x32 MFMA tiles in F32.
//   * setup: the tile's ntaps x 128 neighbour indices go to LDS, the OR of
//     the rows' valid taps is formed (taps no row uses are skipped -- the
//     per-tile offset set of the reference's spconv kernel,
//     cpp_ggml/third_party/sam3d-spconv/src/.../ConvKernel_conv_kernel.cu:
//     62-80), and the referenced source rows are deduplicated with an LDS
//     hash set: a spatially coherent tile references ~3.5 x 128 distinct
//     rows instead of ~21 x 128, so each gathered feature row is fetched
//     once per tile and channel chunk and reused by every tap that needs it.
//   * K loop: for each 64-byte channel chunk, the union of source rows is
//     staged in LDS (row U = zeros for missing taps); then, tap by tap, the
//     weight tile W[co-tile, tap, chunk] streams through a double-buffered
//     LDS stage fed by a 4-step register prefetch ring, one barrier per
//     step, and each lane's A operand is read from its row's union slot.
//     When a tile's union exceeds the stage (poorly ordered rows), the tile
//     falls back to staging each tap's 128 source rows separately.
//   * Q8_0: int8 quants + fp16 block scales are dequantised in registers
//     on their way into LDS: w = bf16(f32(d) * q).
//   * epilogue: + bias in F32, one rounding, direct store of each output
//     row (each output element written exactly once, no atomics).
//   * tiles are mapped XCD-major: workgroup b runs on XCD b % 8, and each
//     XCD receives a contiguous range of row tiles (all N tiles of a row
//     tile together), so a neighbourhood's feature rows stay in that XCD's
//     L2.  LDS stays under 80 KB so two workgroups share a CU.
#include <type_traits>

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
constexpr int kTM = 256;       // output rows per tile
constexpr int kThreads = 512;  // 8 waves
constexpr int kUMax = 1024;    // capacity of the deduplicated source-row stage
constexpr int kHCap = 4096;    // LDS hash-set slots used to deduplicate sources
constexpr int kPD = 4;         // weight-stage prefetch distance (steps)

template <typename T, bool Q8, int TN, int KC, int WM, int WN>
__global__ __launch_bounds__(kThreads, 1) void conv_kernel(ConvArgs a) {
    using M = Mfma<T>;
    constexpr int TM = kTM;
    constexpr int NT = kThreads;
    constexpr int NW = NT / 64;
    constexpr int ES = sizeof(T);
    constexpr int CH = 16 / ES;     // elements per 16-byte chunk
    constexpr int CPR = KC / CH;    // chunks per staged row
    constexpr int PITCH = KC + CH;  // LDS row pitch (elements): +16 bytes against conflicts
    constexpr int B_CHUNKS = TN * CPR;
    constexpr int B_PER_T = (B_CHUNKS + NT - 1) / NT;
    constexpr int WTM = TM / WM;
    constexpr int WTN = TN / WN;
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    static_assert(B_CHUNKS % NT == 0 || B_CHUNKS < NT, "staging geometry");
    static_assert(WM * WN == NW && FM >= 1 && FN >= 1, "wave geometry");
    static_assert(!Q8 || ES == 2, "Q8_0 weights feed 16-bit MFMA operands");
    static_assert((kUMax + 1) * PITCH * ES >= 3 * kHCap * 4, "hash set aliases the A stage");

    __shared__ __attribute__((aligned(16))) T Au[(kUMax + 1) * PITCH];
    __shared__ __attribute__((aligned(16))) T Bs[2 * TN * PITCH];
    __shared__ int32_t sidx[kMaxTaps * TM];  // [tap][row]: union slot, or source row
    __shared__ int32_t urow[kUMax];          // source row of each union slot
    __shared__ int32_t srow[TM];             // output row of each tile row
    __shared__ int32_t taps[kMaxTaps];       // active taps in ascending order
    __shared__ int32_t wsum[NW];
    __shared__ uint32_t smask;
    __shared__ int32_t s_fail;

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
    const int nq = ntaps * TM;

    // setup-phase aliases of the A stage
    int32_t* hkey = reinterpret_cast<int32_t*>(Au);  // source row held by a hash slot
    int32_t* hq = hkey + kHCap;                      // first (tap, row) entry referencing it
    int32_t* hslot = hq + kHCap;                     // its union slot

    if (tid == 0) {
        smask = 0;
        s_fail = 0;
    }
    for (int r = tid; r < TM; r += NT) {
        const int64_t rr = r0 + r;
        int32_t t = -1;
        if (rr < a.n_out) t = a.row_perm ? a.row_perm[rr] : (int32_t)rr;
        if (t >= a.n_out) t = -1;  // a bad permutation entry writes nothing
        srow[r] = t;
    }
    for (int i = tid; i < kHCap; i += NT) {
        hkey[i] = -1;
        hq[i] = INT32_MAX;
    }
    lds_barrier();

    // ---- neighbour indices of the tile and the OR of its valid taps ----
    uint32_t my_mask = 0;
    for (int e = tid; e < nq; e += NT) {
        int r, o;
        if (a.idx_layout == SPC_IDX_TOKEN_MAJOR) {
            r = e / ntaps;
            o = e - r * ntaps;
        } else {
            o = e / TM;
            r = e - o * TM;
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
    for (int off = 32; off > 0; off >>= 1) my_mask |= __shfl_xor(my_mask, off);
    if (lane == 0 && my_mask) atomicOr(&smask, my_mask);
    lds_barrier();

    // ---- deduplicate the sources (LDS hash set).  A spatially coherent tile
    // of 256 rows references ~3.2 x 256 distinct rows instead of ~21 x 256.
    // Union slots are numbered in first-reference order (tap-major, then
    // row), so the rows a wave reads for one tap sit in consecutive slots. ----
    for (int q = tid; q < nq; q += NT) {
        const int32_t src = sidx[q];
        if (src < 0) continue;
        uint32_t h = ((uint32_t)src * 2654435761u) >> (32 - 12);
        bool placed = false;
        for (int it = 0; it < kHCap; ++it) {
            const int32_t prev = atomicCAS(&hkey[h], -1, src);
            if (prev == -1 || prev == src) {
                atomicMin(&hq[h], q);
                sidx[q] = -(int32_t)h - 2;
                placed = true;
                break;
            }
            h = (h + 1) & (kHCap - 1);
        }
        if (!placed) s_fail = 1;
    }
    lds_barrier();
    const int per = (nq + NT - 1) / NT;
    const int qb = min(nq, tid * per);
    const int qe = min(nq, qb + per);
    int cnt = 0;
    for (int q = qb; q < qe; ++q) {
        const int32_t v = sidx[q];
        if (v < -1 && hq[-v - 2] == q) ++cnt;
    }
    int incl = cnt;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    if (lane == 63) wsum[wave] = incl;
    lds_barrier();
    int id = incl - cnt;
    int U = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        if (w < wave) id += wsum[w];
        U += wsum[w];
    }
    const bool fast = !s_fail && U <= kUMax;
    for (int q = qb; q < qe; ++q) {
        const int32_t v = sidx[q];
        if (v < -1 && hq[-v - 2] == q) {
            hslot[-v - 2] = id;
            if (fast) urow[id] = hkey[-v - 2];
            ++id;
        }
    }
    lds_barrier();
    // fast: sidx -> union slot (missing -> zero row U); fallback: raw source
    for (int q = tid; q < nq; q += NT) {
        const int32_t v = sidx[q];
        int32_t out;
        if (v == -1) {
            out = fast ? U : -1;
        } else if (v >= 0) {
            out = v;
        } else {
            out = fast ? hslot[-v - 2] : hkey[-v - 2];
        }
        sidx[q] = out;
    }
    if (tid == 0) {
        int k = 0;
        for (int o = 0; o < ntaps; ++o)
            if ((smask >> o) & 1u) taps[k++] = o;
    }
    lds_barrier();

    const int nt = __popc(smask);
    const int kch = a.cin / KC;
    const int nsteps = nt * kch;  // fast: chunk-major over active taps; fallback: tap-major

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

    // step cursors: (tap index, chunk) of the computed step and of the next
    // weight prefetch; advanced without divisions
    // cursor = tap index | chunk << 8
    auto advance = [&](int c) __attribute__((always_inline)) -> int {
        int t = c & 0xff, kc = c >> 8;
        if (fast) {
            if (++t == nt) {
                t = 0;
                ++kc;
            }
        } else if (++kc == kch) {
            kc = 0;
            ++t;
        }
        return t | (kc << 8);
    };

    struct Slot {
        u32x4 q[B_PER_T];
        float d[Q8 ? B_PER_T : 1];
    };
    Slot ring[kPD];

    auto load_b = [&](int cur, Slot& sl) __attribute__((always_inline)) {
        const int o = taps[cur & 0xff];
        const int kc = cur >> 8;
#pragma unroll
        for (int j = 0; j < B_PER_T; ++j) {
            const int ch = tid + j * NT;
            if (B_CHUNKS < NT && ch >= B_CHUNKS) break;
            const int n = ch / CPR;
            const int seg = ch % CPR;
            const int64_t welem =
                ((int64_t)(co0 + n) * ntaps + o) * a.cin + (int64_t)kc * KC + seg * CH;
            if constexpr (Q8) {
                const u32x2 q = *reinterpret_cast<const u32x2*>(wb + welem);
                sl.q[j] = u32x4{q.x, q.y, 0u, 0u};
                sl.d[j] = f16_bits_to_f32(a.wscale[welem >> 5]);
            } else {
                sl.q[j] = *reinterpret_cast<const u32x4*>(wb + welem * ES);
            }
        }
    };

    auto store_b = [&](int buf, const Slot& sl) __attribute__((always_inline)) {
        T* B = Bs + buf * TN * PITCH;
#pragma unroll
        for (int j = 0; j < B_PER_T; ++j) {
            const int ch = tid + j * NT;
            if (B_CHUNKS < NT && ch >= B_CHUNKS) break;
            const int n = ch / CPR;
            const int seg = ch % CPR;
            if constexpr (Q8) {
                const uint32_t qw[2] = {sl.q[j].x, sl.q[j].y};
                uint32_t packed[4];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t word = qw[h >> 1];
                    const int sh = (h & 1) * 16;
                    const int8_t q0 = (int8_t)((word >> sh) & 0xff);
                    const int8_t q1 = (int8_t)((word >> (sh + 8)) & 0xff);
                    const uint16_t b0 = f32_to_bf16_bits(sl.d[j] * (float)q0);
                    const uint16_t b1 = f32_to_bf16_bits(sl.d[j] * (float)q1);
                    packed[h] = (uint32_t)b0 | ((uint32_t)b1 << 16);
                }
                *reinterpret_cast<u32x4*>(&B[n * PITCH + seg * CH]) =
                    u32x4{packed[0], packed[1], packed[2], packed[3]};
            } else {
                *reinterpret_cast<u32x4*>(&B[n * PITCH + seg * CH]) = sl.q[j];
            }
        }
    };

    // stage the gathered source rows of (tap o, chunk kc) into Au: the whole
    // deduplicated union (fast; row U is the zero row) or the tap's TM rows.
    // All source indices are read first, then all loads issued, then all
    // stores, so a batch's global loads are in flight together.  Missing
    // rows load row 0 (always valid when a step exists) and are zeroed.
    auto stage_a = [&](int o, int kc) __attribute__((always_inline)) {
        const int rows = fast ? U + 1 : TM;
        const int nchunks = rows * CPR;
        const int64_t koff = (int64_t)kc * KC;
        for (int c0 = 0; c0 < nchunks; c0 += NT * 8) {
            int32_t src[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = min(c0 + j * NT + tid, nchunks - 1);
                const int r = c / CPR;
                src[j] = fast ? (r < U ? urow[r] : -1) : sidx[o * TM + r];
            }
            u32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = min(c0 + j * NT + tid, nchunks - 1);
                const int seg = c % CPR;
                const int64_t row = src[j] >= 0 ? src[j] : 0;
                v[j] = *reinterpret_cast<const u32x4*>(xb + (row * a.cin + koff + seg * CH) * ES);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = c0 + j * NT + tid;
                if (c < nchunks) {
                    const int r = c / CPR;
                    const int seg = c % CPR;
                    const u32x4 z = {0u, 0u, 0u, 0u};
                    *reinterpret_cast<u32x4*>(&Au[r * PITCH + seg * CH]) = src[j] >= 0 ? v[j] : z;
                }
            }
        }
    };

    int cc = 0;  // cursor of the step being computed
    int pc = 0;  // cursor of the next weight prefetch

    // Weight ring: B(m) is loaded into ring[m % kPD] at the end of step
    // m-1-kPD and written to LDS at the end of step m-1, so each weight load
    // has kPD steps to land.  The step body is instantiated once per ring
    // position so every slot index is a compile-time constant.
    auto step = [&](int s, auto u_const) __attribute__((always_inline)) {
        constexpr int u = decltype(u_const)::value;
        constexpr int nu = (u + 1) % kPD;
        const int o = taps[cc & 0xff];
        if (fast ? (cc & 0xff) == 0 : true) {
            if (s > 0) lds_barrier();  // every wave is done reading Au
            stage_a(o, cc >> 8);
        }
        lds_barrier();
        // compute step s from Au and Bs[s & 1]
        const T* B = Bs + (s & 1) * TN * PITCH;
        int slot[FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rl = wm * WTM + i * 32 + (lane & 31);
            slot[i] = fast ? sidx[o * TM + rl] : rl;
        }
#pragma unroll
        for (int ks = 0; ks < KC / M::KSUB; ++ks) {
            typename M::frag af[FM];
            typename M::frag bf[FN];
            const int kof = ks * M::KSUB + (lane >> 5) * M::EPL;
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const typename M::frag*>(&Au[slot[i] * PITCH + kof]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *reinterpret_cast<const typename M::frag*>(
                    &B[(wn * WTN + j * 32 + (lane & 31)) * PITCH + kof]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = M::mma(af[i], bf[j], acc[i][j]);
        }
        // weights of step s+1 into the other buffer (its readers, step s-1,
        // finished before this step's barrier); refill that ring slot
        if (s + 1 < nsteps) store_b((s + 1) & 1, ring[nu]);
        if (s + 1 + kPD < nsteps) {
            load_b(pc, ring[nu]);
            pc = advance(pc);
        }
        cc = advance(cc);
    };

    static_assert(kPD == 4, "the prologue and the unrolled loop assume a 4-deep ring");
    if (nsteps > 0) {
        load_b(pc, ring[0]);
        pc = advance(pc);
        store_b(0, ring[0]);
        if (1 < nsteps) { load_b(pc, ring[1]); pc = advance(pc); }
        if (2 < nsteps) { load_b(pc, ring[2]); pc = advance(pc); }
        if (3 < nsteps) { load_b(pc, ring[3]); pc = advance(pc); }
        if (4 < nsteps) { load_b(pc, ring[0]); pc = advance(pc); }
    }
    for (int s0 = 0; s0 < nsteps; s0 += kPD) {
        step(s0, std::integral_constant<int, 0>{});
        if (s0 + 1 < nsteps) step(s0 + 1, std::integral_constant<int, 1>{});
        if (s0 + 2 < nsteps) step(s0 + 2, std::integral_constant<int, 2>{});
        if (s0 + 3 < nsteps) step(s0 + 3, std::integral_constant<int, 3>{});
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

template <typename T, bool Q8, int TN, int KC, int WM, int WN>
hipError_t launch(hipStream_t s, ConvArgs a) {
    const int64_t tiles_m = ceil_div(a.n_out, kTM);
    a.tiles_n = a.cout / TN;
    a.total_tiles = tiles_m * a.tiles_n;
    a.tiles_per_xcd = ceil_div(a.total_tiles, 8);
    const int64_t grid = a.tiles_per_xcd * 8;
    if (grid == 0) return hipSuccess;
    conv_kernel<T, Q8, TN, KC, WM, WN><<<(unsigned)grid, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

// Tile selection: TN = largest of {128, 64, 32} dividing cout; the staged
// row segment is 64 bytes (KC = 32 16-bit or 16 f32 channels).
template <typename T, bool Q8>
hipError_t dispatch(hipStream_t s, const ConvArgs& a) {
    constexpr int KC = 64 / sizeof(T);
    if (a.cout % 128 == 0) return launch<T, Q8, 128, KC, 4, 2>(s, a);
    if (a.cout % 64 == 0) return launch<T, Q8, 64, KC, 8, 1>(s, a);
    return launch<T, Q8, 32, KC, 8, 1>(s, a);
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
