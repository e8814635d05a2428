// conv_kernel.h -- the sparse-convolution kernel (gather -> implicit GEMM on
// CDNA4 matrix cores -> store), instantiated per dtype in conv_*.hip.
//
// Arithmetic contract: the ggml CPU op ggml_compute_forward_sam3d_sparse_
// conv_f16 (PATCH:217-265): y[t,co] = bias[co] + sum over valid taps o and
// channels c of w[co,o,c] * x[idx(t,o),c], accumulated in F32 and rounded
// once to the output dtype.  Taps whose source is outside [0, n_in) add
// nothing (PATCH:255).
//
// Structure (one 8-wave workgroup per 256-row x TN output tile):
//   setup   the tile's NTAPS x 256 neighbour indices are loaded (contiguous,
//           coalesced for the token-major table) into registers; the OR of
//           the valid taps is formed (taps no row uses are skipped -- the
//           per-tile offset set of the reference's spconv kernel,
//           cpp_ggml/third_party/sam3d-spconv/src/.../
//           ConvKernel_conv_kernel.cu:62-80); the referenced source rows are
//           deduplicated with a bitmap over a 32768-row window: a
//           spatially coherent tile references ~3.2 x 256 distinct rows
//           instead of ~21 x 256, and ranks by popcount number them in
//           ascending row order, so the rows one wave reads for one tap sit
//           in consecutive LDS slots.
//   K loop  for each 64-byte channel chunk the union rows are staged once in
//           LDS (slot U = zeros for missing taps); then every wave walks
//           the active taps with no further barrier: its B fragments come
//           straight from global memory (weights prepacked in MFMA fragment
//           order -- one contiguous 1 KB load per fragment, L2-resident),
//           prefetched kPD steps ahead in registers; its A fragments are
//           read from the union slots.
//   Q8_0    int8 quants + per-block scales are dequantised in registers to
//           bf16 operands: w = bf16(f32(d) * q).
//   store   + bias in F32, one rounding, each output row written once.
//   tiles   XCD-major: workgroup b runs on XCD b % 8 and each XCD gets a
//           contiguous range of row tiles, so a neighbourhood's feature rows
//           stay in that XCD's L2.
// Tiles whose union exceeds the stage (rows not spatially ordered) fall
// back to staging each tap's 256 source rows separately.
// NTAPS = 1 with a null map is the dense 1x1x1 conv: row t reads row t.
#pragma once

#include <climits>
#include <type_traits>

#include "common.h"

namespace spc {

struct ConvArgs {
    const void* x;
    const void* w;            // packed or [cout, ntaps, cin]
    const void* wscale;       // Q8_0: packed f32 scales, or fp16 [cout, ntaps, cin/32]
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
    int32_t packed;
    int32_t tiles_n;
    int64_t total_tiles;
    int64_t tiles_per_xcd;
};

// MFMA operand traits per activation type.
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

// Weight-panel geometry shared by the packer and the kernel.  One panel =
// the B operands of (tap, channel chunk, 32 output channels) for all KS
// MFMA k-steps of the chunk, stored lane-major as NG 16-byte words per lane:
// word g of lane l holds k-steps g*G .. g*G+G-1, each EPL elements of
// W[co = 32*c32 + l%32][tap][ci = chunk*KC + ks*KSUB + (l/32)*EPL + e].
template <typename T, bool Q8>
struct Panel {
    static constexpr int KC = 64 / sizeof(T);  // channels per chunk (64-byte rows)
    static constexpr int KSUB = Mfma<T>::KSUB;
    static constexpr int EPL = Mfma<T>::EPL;
    static constexpr int KS = KC / KSUB;                  // MFMA k-steps per chunk
    static constexpr int WB = Q8 ? 1 : (int)sizeof(T);    // stored bytes per weight
    static constexpr int G = 16 / (EPL * WB);             // k-steps per 16-byte word
    static constexpr int NG = KS / G;                     // words per lane per panel
    static_assert(KS % G == 0, "panel geometry");
};

constexpr int kTM = 256;        // output rows per tile
constexpr int kThreads = 512;   // 8 waves
constexpr int kUMax = 1024;     // capacity of the deduplicated source-row stage
constexpr int kWinWords = 1024; // dedupe bitmap: 32768 source rows
constexpr int kPD = 3;          // weight prefetch distance (steps)

template <typename T, bool Q8, bool PACKED, int NTAPS, int TN, int WM, int WN>
__global__ __launch_bounds__(kThreads, 1) void conv_kernel(ConvArgs a) {
    using M = Mfma<T>;
    using P = Panel<T, Q8>;
    constexpr int TM = kTM;
    constexpr int NT = kThreads;
    constexpr int NW = NT / 64;
    constexpr int ES = sizeof(T);
    constexpr int KC = P::KC;
    constexpr int CH = 16 / ES;     // elements per 16-byte chunk
    constexpr int CPR = KC / CH;    // chunks per staged row
    constexpr int PITCH = KC + CH;  // LDS row pitch (elements): +16 bytes against conflicts
    constexpr int WTM = TM / WM;
    constexpr int WTN = TN / WN;
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    constexpr int NQ = NTAPS * TM;
    constexpr int EPT = (NQ + NT - 1) / NT;  // index entries per thread
    static_assert(WM * WN == NW && FM >= 1 && FN >= 1, "wave geometry");
    static_assert(!Q8 || ES == 2, "Q8_0 weights feed 16-bit MFMA operands");
    static_assert((kUMax + 1) * PITCH * ES >= 2 * kWinWords * 4, "bitmap aliases the A stage");
    static_assert(NTAPS <= 32, "tap mask is 32-bit");

    __shared__ __attribute__((aligned(16))) T Au[(kUMax + 1) * PITCH];
    __shared__ int32_t sidx[NQ];      // [tap][row]: union slot, or source row (fallback)
    __shared__ int32_t urow[kUMax];   // source row of each union slot
    __shared__ int32_t srow[TM];      // output row of each tile row
    __shared__ int32_t wsum[NW];
    __shared__ uint32_t smask;
    __shared__ int32_t smin;
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

    uint32_t* bm = reinterpret_cast<uint32_t*>(Au);      // setup-phase aliases
    int32_t* wbase = reinterpret_cast<int32_t*>(Au) + kWinWords;

    if (tid == 0) {
        smask = 0;
        smin = INT_MAX;
        s_fail = 0;
    }
    for (int r = tid; r < TM; r += NT) {
        const int64_t rr = r0 + r;
        int32_t t = -1;
        if (rr < a.n_out) t = a.row_perm ? a.row_perm[rr] : (int32_t)rr;
        if (t >= a.n_out) t = -1;  // a bad permutation entry writes nothing
        srow[r] = t;
    }
    for (int i = tid; i < kWinWords; i += NT) bm[i] = 0u;
    lds_barrier();

    // ---- indices: entry e = r*NTAPS + o, held in registers ----
    const bool contiguous = a.idx_layout == SPC_IDX_TOKEN_MAJOR && a.row_perm == nullptr;
    int32_t ent[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int e = tid + k * NT;
        int32_t src = -1;
        if (e < NQ) {
            const int r = e / NTAPS;
            const int o = e - r * NTAPS;
            if (NTAPS == 1 && a.idx == nullptr) {  // identity map (dense 1x1x1 conv)
                src = srow[r];
            } else if (contiguous) {
                if (r0 + r < a.n_out) src = a.idx[r0 * NTAPS + e];
            } else {
                const int32_t t = srow[r];
                if (t >= 0)
                    src = a.idx_layout == SPC_IDX_TOKEN_MAJOR ? a.idx[(int64_t)t * NTAPS + o]
                                                              : a.idx[(int64_t)o * a.n_out + t];
            }
            if (src < 0 || src >= a.n_in) src = -1;
        }
        ent[k] = src;
    }
    uint32_t my_mask = 0;
    int32_t my_min = INT_MAX;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int e = tid + k * NT;
        if (ent[k] >= 0) {
            my_mask |= 1u << (e % NTAPS);
            my_min = min(my_min, ent[k]);
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        my_mask |= __shfl_xor(my_mask, off);
        my_min = min(my_min, __shfl_xor(my_min, off));
    }
    if (lane == 0) {
        if (my_mask) atomicOr(&smask, my_mask);
        atomicMin(&smin, my_min);
    }
    lds_barrier();

    // ---- dedupe: bitmap over [lo, lo + 32768) ----
    const int32_t lo = smin;
    bool fail = false;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        if (ent[k] >= 0) {
            const int32_t off = ent[k] - lo;
            if (off >= kWinWords * 32) fail = true;
            else atomicOr(&bm[off >> 5], 1u << (off & 31));
        }
    }
    if (fail) s_fail = 1;
    lds_barrier();
    // ranks: thread tid owns words 2*tid, 2*tid+1
    const uint32_t w0 = bm[2 * tid];
    const uint32_t w1 = bm[2 * tid + 1];
    const int cnt = __popc(w0) + __popc(w1);
    int incl = cnt;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    if (lane == 63) wsum[wave] = incl;
    lds_barrier();
    int base = incl - cnt;
    int U = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        if (w < wave) base += wsum[w];
        U += wsum[w];
    }
    const bool fast = !s_fail && U <= kUMax;
    wbase[2 * tid] = base;
    wbase[2 * tid + 1] = base + __popc(w0);
    if (fast) {
        int id = base;
        uint32_t m = w0;
        while (m) {
            const int b = __ffs(m) - 1;
            m &= m - 1;
            urow[id++] = lo + (2 * tid) * 32 + b;
        }
        m = w1;
        while (m) {
            const int b = __ffs(m) - 1;
            m &= m - 1;
            urow[id++] = lo + (2 * tid + 1) * 32 + b;
        }
    }
    lds_barrier();
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int e = tid + k * NT;
        if (e < NQ) {
            const int r = e / NTAPS;
            const int o = e - r * NTAPS;
            int32_t out;
            if (fast) {
                if (ent[k] >= 0) {
                    const int32_t off = ent[k] - lo;
                    const int wi = off >> 5;
                    out = wbase[wi] + __popc(bm[wi] & ((1u << (off & 31)) - 1u));
                } else {
                    out = U;  // the zero row
                }
            } else {
                out = ent[k];
            }
            sidx[o * TM + r] = out;
        }
    }
    lds_barrier();

    const uint32_t tile_mask = smask;
    const int nt = __popc(tile_mask);
    const int kch = a.cin / KC;
    const int nsteps = nt * kch;
    const int ncol32 = a.cout / 32;

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

    // step cursor: (remaining taps of the chunk, chunk); tap = lowest bit
    struct Cursor {
        uint32_t m;
        int kc;
    };
    auto advance = [&](Cursor c) __attribute__((always_inline)) -> Cursor {
        c.m &= c.m - 1;
        if (c.m == 0) {
            c.m = tile_mask;
            ++c.kc;
        }
        return c;
    };

    struct Slot {
        u32x4 q[FN][P::NG];
        float d[Q8 ? FN : 1];
    };
    Slot ring[kPD];

    // B operands of (tap, chunk) for this wave's FN column blocks
    auto load_b = [&](Cursor c, Slot& sl) __attribute__((always_inline)) {
        const int o = __ffs(c.m) - 1;
        const int kc = c.kc;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int c32 = (co0 + wn * WTN) / 32 + j;
            const int co = c32 * 32 + (lane & 31);
            if constexpr (PACKED) {
                const int64_t panel = ((int64_t)o * kch + kc) * ncol32 + c32;
                const u32x4* src = static_cast<const u32x4*>(a.w) + panel * (P::NG * 64);
#pragma unroll
                for (int g = 0; g < P::NG; ++g) sl.q[j][g] = src[g * 64 + lane];
                if constexpr (Q8)
                    sl.d[j] = static_cast<const float*>(a.wscale)[((int64_t)o * kch + kc) * a.cout + co];
            } else {
                const int64_t rowbase = ((int64_t)co * NTAPS + o) * a.cin + (int64_t)kc * KC;
#pragma unroll
                for (int g = 0; g < P::NG; ++g) {
                    if constexpr (P::G == 1) {
                        const int64_t el = rowbase + g * P::KSUB + (lane >> 5) * P::EPL;
                        sl.q[j][g] = *reinterpret_cast<const u32x4*>(
                            static_cast<const char*>(a.w) + el * P::WB);
                    } else {
                        uint32_t words[4];
                        constexpr int WPK = 4 / P::G;  // 32-bit words per k-step
#pragma unroll
                        for (int i = 0; i < P::G; ++i) {
                            const int ks = g * P::G + i;
                            const int64_t el = rowbase + ks * P::KSUB + (lane >> 5) * P::EPL;
                            const uint32_t* wp = reinterpret_cast<const uint32_t*>(
                                static_cast<const char*>(a.w) + el * P::WB);
#pragma unroll
                            for (int h = 0; h < WPK; ++h) words[i * WPK + h] = wp[h];
                        }
                        sl.q[j][g] = u32x4{words[0], words[1], words[2], words[3]};
                    }
                }
                if constexpr (Q8)
                    sl.d[j] = f16_bits_to_f32(static_cast<const uint16_t*>(a.wscale)[rowbase >> 5]);
            }
        }
    };

    // B fragment of k-step ks from a prefetched slot
    auto b_frag = [&](const Slot& sl, int j, int ks) __attribute__((always_inline)) {
        typename M::frag f;
        const u32x4 wv = sl.q[j][ks / P::G];
        if constexpr (Q8) {
            // 8 int8 quants of this k-step -> bf16(d * q)
            const uint32_t lo32 = (ks % P::G) == 0 ? wv.x : wv.z;
            const uint32_t hi32 = (ks % P::G) == 0 ? wv.y : wv.w;
            uint16_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t word = e < 4 ? lo32 : hi32;
                const int8_t q = (int8_t)((word >> (8 * (e & 3))) & 0xff);
                h[e] = f32_to_bf16_bits(sl.d[j] * (float)q);
            }
            const u32x4 pk = {(uint32_t)h[0] | ((uint32_t)h[1] << 16),
                              (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                              (uint32_t)h[4] | ((uint32_t)h[5] << 16),
                              (uint32_t)h[6] | ((uint32_t)h[7] << 16)};
            f = __builtin_bit_cast(typename M::frag, pk);
        } else if constexpr (P::G == 1) {
            f = __builtin_bit_cast(typename M::frag, wv);
        } else {
            // explicit component select: indexing the vector by (ks % G) read
            // component 0 for every k-step in generated code
            const int c = ks % P::G;
            const uint32_t word = c == 0 ? wv.x : c == 1 ? wv.y : c == 2 ? wv.z : wv.w;
            f = __builtin_bit_cast(float, word);
        }
        return f;
    };

    // stage the gathered source rows of (tap o, chunk kc) into Au: the whole
    // deduplicated union (fast; slot U is the zero row) or the tap's TM
    // rows.  All indices first, then all loads, then all stores, so a
    // batch's global loads are in flight together; missing rows load row 0
    // (valid whenever a step exists) and are zeroed.
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

    Cursor cc{tile_mask, 0};  // step being computed
    Cursor pc{tile_mask, 0};  // next weight prefetch

    // Weight ring: the operands of step m are loaded into ring[m % kPD]
    // during step m - kPD; the step body is instantiated once per ring
    // position so every slot index is a compile-time constant.
    // A operands of one step: union slots of the wave's rows for a tap, and
    // the fragments read from them.  Slots depend only on the tap, so they
    // are read two steps ahead; fragments one step ahead (within a chunk),
    // overlapping the LDS latency with the current step's MFMAs.
    typedef typename M::frag AFrag[P::KS][FM];
    auto read_slots = [&](int o, int* sl) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rl = wm * WTM + i * 32 + (lane & 31);
            sl[i] = fast ? sidx[o * TM + rl] : rl;
        }
    };
    auto read_frags = [&](const int* sl, AFrag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < P::KS; ++ks) {
            const int kof = ks * M::KSUB + (lane >> 5) * M::EPL;
#pragma unroll
            for (int i = 0; i < FM; ++i)
                f[ks][i] = *reinterpret_cast<const typename M::frag*>(&Au[sl[i] * PITCH + kof]);
        }
    };
    AFrag afc;         // fragments of the current step
    int slot_n[FM];    // slots of the next step

    auto step = [&](int s, auto u_const) __attribute__((always_inline)) {
        constexpr int u = decltype(u_const)::value;
        const int o = __ffs(cc.m) - 1;
        const Cursor nc = advance(cc);  // step s+1
        if (fast ? cc.m == tile_mask : true) {  // first tap of a chunk, or every step
            if (s > 0) lds_barrier();           // every wave is done reading Au
            stage_a(o, cc.kc);
            lds_barrier();
            int sl[FM];
            read_slots(o, sl);
            read_frags(sl, afc);
            if (s + 1 < nsteps) read_slots(__ffs(nc.m) - 1, slot_n);
        }
        // prefetch: fragments of step s+1 (same chunk) and slots of step s+2
        const bool next_same_chunk = fast && s + 1 < nsteps && nc.kc == cc.kc;
        AFrag afn;
        if (next_same_chunk) read_frags(slot_n, afn);
        int slot_nn[FM];
        if (s + 2 < nsteps) read_slots(__ffs(advance(nc).m) - 1, slot_nn);
#pragma unroll
        for (int ks = 0; ks < P::KS; ++ks) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const typename M::frag bf = b_frag(ring[u], j, ks);
#pragma unroll
                for (int i = 0; i < FM; ++i) acc[i][j] = M::mma(afc[ks][i], bf, acc[i][j]);
            }
        }
        if (next_same_chunk) {
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks)
#pragma unroll
                for (int i = 0; i < FM; ++i) afc[ks][i] = afn[ks][i];
        }
        if (s + 2 < nsteps) {
#pragma unroll
            for (int i = 0; i < FM; ++i) slot_n[i] = slot_nn[i];
        }
        if (s + kPD < nsteps) {
            load_b(pc, ring[u]);
            pc = advance(pc);
        }
        cc = nc;
    };

    static_assert(kPD == 3, "the prologue and the unrolled loop assume a 3-deep ring");
    if (nsteps > 0) {
        load_b(pc, ring[0]);
        pc = advance(pc);
        if (1 < nsteps) {
            load_b(pc, ring[1]);
            pc = advance(pc);
        }
        if (2 < nsteps) {
            load_b(pc, ring[2]);
            pc = advance(pc);
        }
    }
    for (int s0 = 0; s0 < nsteps; s0 += kPD) {
        step(s0, std::integral_constant<int, 0>{});
        if (s0 + 1 < nsteps) step(s0 + 1, std::integral_constant<int, 1>{});
        if (s0 + 2 < nsteps) step(s0 + 2, std::integral_constant<int, 2>{});
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

template <typename T, bool Q8, bool PACKED, int NTAPS, int TN, int WM, int WN>
hipError_t launch_conv(hipStream_t s, ConvArgs a) {
    const int64_t tiles_m = ceil_div(a.n_out, kTM);
    a.tiles_n = a.cout / TN;
    a.total_tiles = tiles_m * a.tiles_n;
    a.tiles_per_xcd = ceil_div(a.total_tiles, 8);
    const int64_t grid = a.tiles_per_xcd * 8;
    if (grid == 0) return hipSuccess;
    conv_kernel<T, Q8, PACKED, NTAPS, TN, WM, WN><<<(unsigned)grid, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

// TN = largest of {128, 64, 32} dividing cout; 8 waves as 4x2 (64x64 wave
// tiles) or 8x1.
template <typename T, bool Q8, bool PACKED, int NTAPS>
hipError_t dispatch_tn(hipStream_t s, const ConvArgs& a) {
    if (a.cout % 128 == 0) return launch_conv<T, Q8, PACKED, NTAPS, 128, 4, 2>(s, a);
    if (a.cout % 64 == 0) return launch_conv<T, Q8, PACKED, NTAPS, 64, 8, 1>(s, a);
    return launch_conv<T, Q8, PACKED, NTAPS, 32, 8, 1>(s, a);
}

template <typename T, bool Q8>
hipError_t dispatch_conv(hipStream_t s, const ConvArgs& a) {
    if (a.ntaps == 27)
        return a.packed ? dispatch_tn<T, Q8, true, 27>(s, a) : dispatch_tn<T, Q8, false, 27>(s, a);
    if (a.ntaps == 8)
        return a.packed ? dispatch_tn<T, Q8, true, 8>(s, a) : dispatch_tn<T, Q8, false, 8>(s, a);
    if (a.ntaps == 1)
        return a.packed ? dispatch_tn<T, Q8, true, 1>(s, a) : dispatch_tn<T, Q8, false, 1>(s, a);
    return hipErrorInvalidValue;
}

// per-dtype instantiations (conv_bf16.hip, conv_f16.hip, conv_f32.hip, conv_q8.hip)
hipError_t conv_bf16(hipStream_t s, const ConvArgs& a);
hipError_t conv_f16(hipStream_t s, const ConvArgs& a);
hipError_t conv_f32(hipStream_t s, const ConvArgs& a);
hipError_t conv_q8(hipStream_t s, const ConvArgs& a);

}  // namespace spc
