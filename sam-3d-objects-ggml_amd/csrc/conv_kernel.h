// conv_kernel.h -- the sparse-convolution kernel (gather -> implicit GEMM on
// CDNA4 matrix cores -> store), instantiated per dtype in conv_*.hip.
//
// Arithmetic contract: the ggml CPU op ggml_compute_forward_sam3d_sparse_
// conv_f16 (PATCH:217-265): y[t,co] = bias[co] + sum over valid taps o and
// channels c of w[co,o,c] * x[idx(t,o),c], accumulated in F32 and rounded
// once to the output dtype.  Taps whose source is outside [0, n_in) add
// nothing (PATCH:255).
//
// Structure (one 8-wave workgroup -- two waves per SIMD -- per 256-row x TN
// output tile; with TN = 128 each wave owns a 64 x 64 block of F32
// accumulators):
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
//           in nearly consecutive LDS slots.
//   K loop  channels are consumed in 64-byte chunks.  A chunk's union rows
//           live in one of two LDS buffers (slot U = zeros for missing
//           taps); while the waves run the MFMAs of chunk kc over all active
//           taps, LDS-DMA loads (buffer_load_dwordx4 ... lds) fill the other
//           buffer with the next chunk, so one barrier per chunk is the
//           only synchronisation.  B fragments come straight from global
//           memory (weights prepacked in MFMA fragment order -- one
//           contiguous 1 KB load per fragment, L2-resident) through a
//           register ring PD steps deep; A fragments and their slots are
//           read from LDS one and two steps ahead.
//   Q8_0    int8 quants + per-block scales are dequantised in registers to
//           bf16 operands: w = bf16(f32(d) * q).
//   store   + bias in F32, one rounding; the MFMAs produce the transposed
//           tile, so each lane holds runs of consecutive output channels of
//           one row: they pass through an LDS output tile and every output
//           row is written once with coalesced 16-byte stores (8-wave
//           16-bit tiles: per wave, through a private LDS region, with no
//           workgroup barrier).
//   shapes  the tile geometry (Geo below) sets rows per tile, stage rows
//           and buffers: 256-row double-buffered tiles for long convs,
//           128-row single-buffered ones several to a CU for short tiles,
//           256-row single-buffered ones for one-chunk rows, and 64-row
//           four-buffer ones for the stride-2 conv; every geometry runs the
//           same MFMA steps in the same order, so all give the same bits.
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
    int32_t col_major;        // full row tiles' tiles taken column tile by column tile
    int64_t total_tiles;
    int64_t heavy_tiles;      // tiles of full row tiles (mapped XCD-major)
    int64_t class_rows;       // > 0: rows [c * class_rows, (c + 1) * class_rows) use weight
    int32_t n_classes;        //   taps c * ntaps .. (packed weights of n_classes * ntaps taps)
    int64_t tiles_per_xcd;
    const void* plan;         // per-row-tile setup from conv_plan_kernel, or null
    // Self-refreshing plan (with plan, natural row order): plan_dirty holds
    // one flag per (128 output rows, tap), set where the index entries
    // differ from those the plan was built from (idx_cache, same layout as
    // idx; flag 27 f + o for rows [128 f, 128 f + 128) and tap o).  A tile
    // over flagged rows sets itself up instead of reading its plan tile, and
    // its first column tile writes the plan tile and the entries back.
    const int32_t* plan_dirty;
    int32_t* idx_cache;
    int32_t num_cu;           // compute units of the device (tile-width choice)
    // fused epilogue (spc_conv_epilogue): SPC_EPI_NONE / _RESIDUAL / _NORM_MOD_SILU
    int32_t epi_mode;
    float epi_eps;
    const void* residual;     // [n_out, cout] in the feature dtype, or [n_residual, cout]
    const int32_t* residual_rows;  // optional residual row of each output row
    int64_t n_residual;
    const float* epi_scale;   // [n_batch, cout]
    const float* epi_shift;   // [n_batch, cout]
    const int32_t* coords;    // [n_out, 4]: batch of each output row
    int64_t n_batch;          // rows of epi_scale / epi_shift
    int32_t geometry;         // tile geometry: 0 by shape, 1 wide, 2 small
};

// MFMA operand traits per activation type.  The conv computes transposed
// blocks: the weights are the MFMA's row operand (BC output channels) and the
// gathered features its column operand (BR output rows), so a lane's
// accumulators hold runs of consecutive channels of one output row.
//   16-bit  v_mfma_f32_16x16x32_{bf16,f16}: 16 rows x 16 channels per block,
//           the 32 channels of a 64-byte chunk in one instruction; lane l
//           supplies 8 consecutive channels 8 (l / 16) .. of row / output
//           channel l % 16 and holds channels 4 (l / 16) .. + 3 of row l % 16.
//           (Under full-chip load with real data this shape sustains ~2.0
//           PFLOP/s against ~1.75 for 32x32x16: at equal work it draws less
//           power, and the chip holds a higher clock.)
//   f32     v_mfma_f32_32x32x2f32: 32 x 32 blocks, two channels per k-step;
//           lane l holds channels 8 g + 4 (l / 32) .. + 3 (g < 4) of row l % 32.
template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
    static constexpr int KSUB = 32;  // K per instruction
    static constexpr int EPL = 8;    // elements per lane per operand
    static constexpr int BR = 16;    // output rows per block
    static constexpr int BC = 16;    // output channels per block
    static constexpr int NRUN = 1;   // runs of four channels per lane per block
    typedef bf16x8 frag;
    typedef floatx4 acc_t;
    __device__ static acc_t mma(frag a, frag b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // first channel (within the block) of a lane's run g
    __host__ __device__ static constexpr int run(int lane, int) { return 4 * (lane >> 4); }
    __device__ static uint16_t cvt(float v) { return f32_to_bf16_bits(v); }
    __device__ static float ld(const void* p, int64_t i) {
        return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
    __device__ static float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
    __device__ static float unpack(uint32_t w, int h) { return __uint_as_float(h ? w & 0xffff0000u : w << 16); }
};

template <>
struct Mfma<_Float16> {
    static constexpr int KSUB = 32;
    static constexpr int EPL = 8;
    static constexpr int BR = 16;
    static constexpr int BC = 16;
    static constexpr int NRUN = 1;
    typedef f16x8 frag;
    typedef floatx4 acc_t;
    __device__ static acc_t mma(frag a, frag b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    __host__ __device__ static constexpr int run(int lane, int) { return 4 * (lane >> 4); }
    __device__ static uint16_t cvt(float v) { return f32_to_f16_bits(v); }
    __device__ static float ld(const void* p, int64_t i) {
        return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
    __device__ static float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
    __device__ static float unpack(uint32_t w, int h) { return f16_bits_to_f32((uint16_t)(h ? w >> 16 : w)); }
};

template <>
struct Mfma<float> {
    static constexpr int KSUB = 2;
    static constexpr int EPL = 1;
    static constexpr int BR = 32;
    static constexpr int BC = 32;
    static constexpr int NRUN = 4;
    typedef float frag;
    typedef floatx16 acc_t;
    __device__ static acc_t mma(frag a, frag b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __host__ __device__ static constexpr int run(int lane, int g) { return 8 * g + 4 * (lane >> 5); }
    __device__ static float cvt(float v) { return v; }
    __device__ static float ld(const void* p, int64_t i) {
        return static_cast<const float*>(p)[i];
    }
    __device__ static float round(float v) { return v; }
};

// Weight-panel geometry shared by the packers and the kernel.  One panel =
// the row operands of (tap, channel chunk, 32 output channels): NF = KS x NH
// MFMA fragments (KS k-steps of the chunk, NH = 32 / BC channel blocks),
// fragment f = ks NH + h holding, for lane l, EPL elements of
// W[co = 32 c32 + h BC + l % BC][tap][ci = chunk KC + ks KSUB + (l / BC) EPL + e].
// Stored lane-major as NG 16-byte words per lane, G fragments per word
// (16-bit: two words, one per 16-channel block; Q8_0: one word, both blocks'
// 8 quants; f32: two words of four k-steps each).
template <typename T, bool Q8>
struct Panel {
    static constexpr int KC = 64 / sizeof(T);  // channels per chunk (64-byte rows)
    static constexpr int KSUB = Mfma<T>::KSUB;
    static constexpr int EPL = Mfma<T>::EPL;
    static constexpr int BC = Mfma<T>::BC;
    static constexpr int KS = KC / KSUB;                  // MFMA k-steps per chunk
    static constexpr int NH = 32 / BC;                    // channel blocks per panel
    static constexpr int NF = KS * NH;                    // fragments per panel
    static constexpr int WB = Q8 ? 1 : (int)sizeof(T);    // stored bytes per weight
    static constexpr int G = 16 / (EPL * WB);             // fragments per 16-byte word
    static constexpr int NG = NF / G;                     // words per lane per panel
    static_assert(NF % G == 0 && KS * KSUB == KC && NH * BC == 32, "panel geometry");
    // output channel (within the panel) and first input channel (within the
    // chunk) of lane l's elements of fragment f
    __host__ __device__ static constexpr int co_of(int f, int lane) { return (f % NH) * BC + lane % BC; }
    __host__ __device__ static constexpr int ci_of(int f, int lane) { return (f / NH) * KSUB + (lane / BC) * EPL; }
};

// Q8_0 dequantisation of one k-step's 8 quants (byte e of lo, hi = quant
// e, e+4) with block scale d: bf16(d * q), rounded to nearest even.  The
// bytes are biased to unsigned (u = q + 128, one xor per word) so each
// converts with a single unsigned-byte convert; fma(d, u, -128 d) is exactly
// d * q (d is an fp16 value and |q| <= 127, so every intermediate is exact in
// F32).  The conv's in-register path and the panel expander both use it, so
// they agree bit for bit.
__device__ __forceinline__ bf16x8 q8_dequant8(uint32_t lo, uint32_t hi, float d) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    const float nb = -128.0f * d;
    bf16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t word = e < 4 ? lo : hi;
        f[e] = (__bf16)__builtin_fmaf(d, (float)((word >> (8 * (e & 3))) & 0xffu), nb);
    }
    return f;
}

// The same dequantisation rounded to f16: f16(f32(d) * q), the operand the
// reference's Q8_0 convs feed their f16 GEMM (as_f16, SRC/slat_flow_graph.
// cpp:24-27; as_f32 then the F16 weight view, SRC/mesh_decoder_graph.cpp:
// 309-312).  d * q is exact in F32; one round-to-nearest-even to f16.
__device__ __forceinline__ f16x8 q8_dequant8_f16(uint32_t lo, uint32_t hi, float d) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    const float nb = -128.0f * d;
    f16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t word = e < 4 ? lo : hi;
        f[e] = (_Float16)__builtin_fmaf(d, (float)((word >> (8 * (e & 3))) & 0xffu), nb);
    }
    return f;
}

constexpr int kWinWords = 1024;  // dedupe bitmap: 32768 source rows
// Tiles whose sources span more take a bitmap over 65536 rows, and only
// tiles beyond that the LDS hash: the sources of a 256-row tile of the
// 1,393,024-row 256^3 subdivided shell (children in parent-major order)
// span up to 64,532 rows, and 5,273 of its 5,442 tiles exceed 32768 (that
// level's tile plan: 314 us through the hash, 215 us with a 65536-row
// bitmap for every tile -- which costs the tiles that fit 32768 rows 14 ->
// 16 us a plan, so the window is chosen per tile from the span).
constexpr int kWinWordsWide = 2048;
constexpr int kHashBits = 11;    // wider spans: LDS hash of the tile's source rows
constexpr int kHashSlots = 1 << kHashBits;  // 64-bit slots: row | rank << 32
constexpr int kSortCap = 1024;   // distinct rows collected after hashing (> any stage's UMAX)
constexpr int kSetupScratchWords = 2 * kWinWordsWide > 2 * kHashSlots + 2 * kSortCap
                                       ? 2 * kWinWordsWide
                                       : 2 * kHashSlots + 2 * kSortCap;
constexpr int kSegs = 4;        // 16-byte segments per staged 64-byte row chunk

// Tile geometry: TM output rows per tile, a deduplicated source-row stage of
// UMAX rows (+ the zero row), NBUF A buffers, and the staged row layout.
//   GeoWide   256 rows, 895-row stage, double-buffered (the next chunk lands
//             while the MFMAs run), 64-byte rows with swizzled segments:
//             112 KB of A stage, one workgroup of 8 waves per CU -- the wide
//             convs, where every tile is long.
//   GeoSmall  128 rows (64 for the 8-tap stride-2 conv, whose 128 coarse
//             rows reference ~680 fine rows), 511-row stage, swizzled rows,
//             one buffer: ~42 KB of LDS, three workgroups of 4 waves per CU,
//             which hide each other's staging and setup latency -- the short
//             tiles of small channel counts, small row counts and stride-2.
//             (A double-buffered variant measured no faster: stride-2
//             128 -> 128 11.6 -> 11.5 us, subdivided 128^3 C=64 24.7 -> 27.4
//             us with two workgroups per CU instead of three.)
//   GeoTall   256 rows over one 559-row stage (the most that keeps three
//             workgroups of 4 waves per CU: ~53 KB of LDS each), twice the
//             rows in flight per CU of GeoSmall -- rows of one 64-byte chunk,
//             whose tiles are mostly setup and staging latency and whose
//             256-row union fits on surface-like sets (the subdivided 256^3
//             shell: 429 rows on average, 523 at most).  It reads the wide
//             tiles' plans (same row tiles, slot keys and plan layout); a tile
//             whose union exceeds its stage takes the per-tap fallback, two
//             taps per round, about four times the staged tile's time.
//   GeoQuad   GeoSmall<8>'s 64-row tiles and plan over four 511-row buffers
//             (128 KB, one workgroup per CU): a tile stages four channel
//             chunks at once, so a stride-2 conv over 16-bit rows of up to
//             128 channels waits for one staging instead of one per chunk --
//             for the stride-2 convs whose tiles fit the device in one round.
// Staged row layouts (one 64-byte chunk of a union row = four 16-byte
// segments; a 16-bit wave's feature-fragment read takes all four segments
// of 16 slots, lane l segment l / 16 of slot l % 16):
//   SW = false  row r at an 80-byte pitch: segment s at unit 5r + s.
//   SW = true   row r at a 64-byte pitch, segment s at unit 4r + (s ^ ((r >> 1)
//               & 3)): 16 consecutive slots read that way are served at the
//               LDS's full 198 B/clk per CU (an LDS probe, 8 waves per CU:
//               swizzling on row bits 2-3 instead -- conflict-free for the
//               32-row reads of a 32x32 MFMA operand -- gives 128 B/clk for
//               this pattern, no swizzle 128 B/clk; the f32 kernels' 4-byte
//               reads take the same time either way).
// A slot key is the unit of segment 0's position base: unit(s) = key + s
// (padded) or key ^ s (swizzled: the key's low two bits carry the swizzle).
// A tap's slot keys sit in 64-row groups, row r of a group at position
// 4 (r % 16) + r / 16, so the 16-bit kernels' four keys of lane l (rows
// l % 16 + 16 i of a 64-row wave tile) are one 8-byte LDS read.
template <int TM_, int UMAX_, int NBUF_, bool SW_, int PUMAX_ = UMAX_>
struct Geo {
    static constexpr int TM = TM_;
    static constexpr int UMAX = UMAX_;
    static constexpr int NBUF = NBUF_;
    static constexpr bool SW = SW_;
    static constexpr int PITCH = SW ? 4 : 5;            // 16-byte units per staged row
    static constexpr int UROWCAP = (UMAX + 3) / 4 * 4;  // union-row table (16-byte multiple)
    static constexpr int PUROWCAP = (PUMAX_ + 3) / 4 * 4;  // the plan's union-row table
    // the plan section the geometry reads: the 256-row tiles' (up to 895
    // union rows) or the small tiles'
    static constexpr bool WIDE_PLAN = TM_ == 256 && PUMAX_ == 895;
    // 16-byte units per A buffer: whole 64-unit blocks (one LDS-DMA
    // instruction each) holding the UMAX union rows and the zero row
    static constexpr int STAGE = ((UMAX + 1) * PITCH + 63) / 64 * 64;
    __host__ __device__ static constexpr int swz(int r) { return (r >> 1) & 3; }
    __host__ __device__ static constexpr int key(int r) { return SW ? 4 * r + swz(r) : 5 * r; }
    __host__ __device__ static constexpr int unit(int k, int s) { return SW ? (k ^ s) : k + s; }
    __host__ __device__ static constexpr int seg_pos(int r, int s) { return unit(key(r), s); }
    // One row tile's plan: header (U, tap mask, fast flag, tap words),
    // output rows, union rows, slot keys.  It depends only on the index
    // table, its layout, the row order and NTAPS -- not on channels or
    // weights.
    static constexpr int PLAN_SROW = 64;
    static constexpr int PLAN_UROW = PLAN_SROW + 4 * TM;
    static constexpr int PLAN_SIDX = PLAN_UROW + 4 * PUROWCAP;
    __host__ __device__ static constexpr int64_t plan_tile_bytes(int ntaps) {
        return (PLAN_SIDX + 2 * (int64_t)(ntaps + 1) * TM + 255) / 256 * 256;
    }
};
using GeoWide = Geo<256, 895, 2, true>;
template <int NTAPS>
using GeoSmall = Geo<NTAPS == 8 ? 64 : 128, 511, 1, true>;
using GeoTall = Geo<256, 559, 1, true, 895>;
using GeoQuad = Geo<64, 511, 4, true>;
static_assert(GeoWide::STAGE == 3584 && GeoSmall<27>::STAGE == 2048 && GeoTall::STAGE == 2240,
              "stage geometry");
static_assert(GeoQuad::plan_tile_bytes(8) == GeoSmall<8>::plan_tile_bytes(8) && !GeoQuad::WIDE_PLAN,
              "the four-buffer tiles read the small plan");
static_assert(GeoTall::WIDE_PLAN && GeoTall::plan_tile_bytes(27) == GeoWide::plan_tile_bytes(27) &&
                  GeoTall::PLAN_SIDX == GeoWide::PLAN_SIDX && !GeoSmall<27>::WIDE_PLAN,
              "the tall tiles read the wide plan");

// Plan buffer: the GeoWide plan of every 256-row tile, then the GeoSmall
// plan of every small tile (a conv picks its geometry by shape).
__host__ __device__ constexpr int64_t plan_wide_bytes(int64_t n_out, int ntaps) {
    return (n_out + GeoWide::TM - 1) / GeoWide::TM * GeoWide::plan_tile_bytes(ntaps);
}
__host__ __device__ constexpr int64_t plan_small_bytes(int64_t n_out, int ntaps) {
    return ntaps == 8 ? (n_out + 63) / 64 * GeoSmall<8>::plan_tile_bytes(8)
                      : (n_out + 127) / 128 * GeoSmall<27>::plan_tile_bytes(ntaps);
}

constexpr int kTapWords = 8;  // step taps, four per word: up to 28 steps per chunk
constexpr int32_t kPlanMagic = 0x314e4c50;  // header word 3 of every built plan tile

// Position of tile row r among a tap's TM slot keys: 64-row groups, row
// 16 i + j of a group at 4 j + i.
__host__ __device__ constexpr int slot_pos(int r) { return (r & ~63) | ((r & 15) << 2) | ((r >> 4) & 3); }

// Shared-memory arrays of one tile's setup.
struct TileLds {
    uint32_t* scratch;  // kSetupScratchWords words: dedupe bitmap + word ranks, or the hash
    uint16_t* sidx;     // (NTAPS + 1) x TM slot keys; row NTAPS = the zero slot
    uint32_t* tlw;      // kTapWords
    int32_t* urow;      // UMAX source rows of the union slots
    int32_t* srow;      // TM output rows of the tile rows
    int32_t* wsum;      // one per wave
    int32_t* misc;      // [0] tap mask [1] min source row [2] unused [3] U [4] fast
                        // [5] distinct rows (hash path) [6] max source row
};

// Tile setup: the tile's NTAPS x 256 neighbour indices are loaded
// (contiguous, coalesced for the token-major table) into registers; the OR
// of the valid taps is formed (taps no row uses are skipped -- the per-tile
// offset set of the reference's spconv kernel, cpp_ggml/third_party/
// sam3d-spconv/src/.../ConvKernel_conv_kernel.cu:62-80); the referenced
// source rows are deduplicated with a bitmap over a 32768-row window (then a
// 65536-row one, then an LDS hash, for tiles whose sources span more): a
// spatially coherent tile references ~3.2 x 256 distinct rows instead of
// ~21 x 256, and ranks by popcount number them in ascending row order.
// Ends with a barrier; results in L (misc[0], misc[3], misc[4]).
template <int NTAPS, int NT, int PD, typename GEO>
__device__ __forceinline__ void tile_setup(const ConvArgs& a, int64_t r0, const TileLds& L) {
    constexpr int TM = GEO::TM;
    constexpr int kUMax = GEO::UMAX;
    constexpr int NW = NT / 64;
    constexpr int NQ = NTAPS * TM;
    constexpr int EPT = (NQ + NT - 1) / NT;
    static_assert(kWinWords % NT == 0 && kWinWordsWide % NT == 0, "setup geometry");
    static_assert((NTAPS + PD - 1) / PD < kTapWords, "tap words");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t* bm = L.scratch;

    if (tid == 0) {
        L.misc[0] = 0;
        L.misc[1] = INT_MAX;
        L.misc[2] = 0;
        L.misc[6] = INT_MIN;
    }
    for (int r = tid; r < TM; r += NT) {
        const int64_t rr = r0 + r;
        int32_t t = -1;
        if (rr < a.n_out) t = a.row_perm ? a.row_perm[rr] : (int32_t)rr;
        if (t >= a.n_out) t = -1;  // a bad permutation entry writes nothing
        L.srow[r] = t;
    }
    for (int i = tid; i < kWinWordsWide; i += NT) bm[i] = 0u;  // either window
    lds_barrier();

    const bool contiguous = a.idx_layout == SPC_IDX_TOKEN_MAJOR && a.row_perm == nullptr;
    int32_t ent[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int e = tid + k * NT;
        int32_t src = -1;
        if (e < NQ) {
            const int r = e / NTAPS;
            const int o = e - r * NTAPS;
            if (contiguous && a.idx != nullptr) {
                if (r0 + r < a.n_out) src = a.idx[r0 * NTAPS + e];
            } else {
                const int32_t t = L.srow[r];
                if (t >= 0) {
                    if (NTAPS == 1 && a.idx == nullptr) src = t;  // identity map (dense 1x1x1)
                    else if (a.idx_layout == SPC_IDX_TOKEN_MAJOR) src = a.idx[(int64_t)t * NTAPS + o];
                    else src = a.idx[(int64_t)o * a.n_out + t];
                }
            }
            if (src < 0 || src >= a.n_in) src = -1;
        }
        ent[k] = src;
    }
    uint32_t my_mask = 0;
    int32_t my_min = INT_MAX, my_max = INT_MIN;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        const int e = tid + k * NT;
        if (ent[k] >= 0) {
            my_mask |= 1u << (e % NTAPS);
            my_min = min(my_min, ent[k]);
            my_max = max(my_max, ent[k]);
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        my_mask |= __shfl_xor(my_mask, off);
        my_min = min(my_min, __shfl_xor(my_min, off));
        my_max = max(my_max, __shfl_xor(my_max, off));
    }
    if (lane == 0) {
        if (my_mask) atomicOr(reinterpret_cast<uint32_t*>(&L.misc[0]), my_mask);
        atomicMin(&L.misc[1], my_min);
        atomicMax(&L.misc[6], my_max);
    }
    lds_barrier();

    // ---- dedupe: a bitmap over [lo, lo + 32768), or [lo, lo + 65536) when
    // the sources span more, or the LDS hash beyond that ----
    const int32_t lo = L.misc[1];
    const int64_t span = (int64_t)L.misc[6] - lo + 1;  // <= 0 without sources
    const bool wide = span > kWinWords * 32;
    const bool hashed = span > kWinWordsWide * 32;
    if (!hashed) {
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            if (ent[k] >= 0) {
                const int32_t off = ent[k] - lo;  // < span by the reduction
                atomicOr(&bm[off >> 5], 1u << (off & 31));
            }
        }
        lds_barrier();
    }
    int U;
    bool fast;
    if (hashed) {
        // ---- the sources span more than the window (large tensors whose
        // neighbour slabs lie far apart in row order): insert them into an
        // LDS hash table (64-bit slots, linear probing), collect the distinct
        // rows, place each at its rank among them (a count of smaller rows,
        // read by all lanes at once) and store the rank in its slot; every
        // entry then finds its rank in its slot -- the same ascending union
        // as the bitmap gives.  Inserting stops once kSortCap distinct rows
        // are in (the tile is then not staged), so at most kSortCap + NT
        // slots are ever taken and every probe ends at an empty slot.
        static_assert(kHashSlots > kSortCap + NT && kSortCap > kUMax, "hash geometry");
        unsigned long long* ht = reinterpret_cast<unsigned long long*>(L.scratch);
        int32_t* ul = reinterpret_cast<int32_t*>(ht + kHashSlots);  // distinct rows
        int32_t* us = ul + kSortCap;                                 // their slots
        constexpr unsigned long long kEmpty = ~0ull;
        for (int i = tid; i < kHashSlots; i += NT) ht[i] = kEmpty;
        if (tid == 0) L.misc[5] = 0;
        lds_barrier();
        volatile int32_t* ndist = &L.misc[5];
        auto hash = [](int32_t key) { return ((uint32_t)key * 2654435761u) >> (32 - kHashBits); };
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const int32_t key = ent[k];
            if (key >= 0) {
                uint32_t h = hash(key);
                for (int probe = 0; probe < kHashSlots && *ndist < kSortCap; ++probe) {
                    const unsigned long long prev = atomicCAS(&ht[h], kEmpty, (unsigned long long)(uint32_t)key);
                    if (prev == kEmpty) {
                        const int i = atomicAdd(&L.misc[5], 1);
                        if (i < kSortCap) {
                            ul[i] = key;
                            us[i] = (int32_t)h;
                        }
                        break;
                    }
                    if ((uint32_t)prev == (uint32_t)key) break;
                    h = (h + 1) & (kHashSlots - 1);
                }
            }
        }
        lds_barrier();
        U = L.misc[5];
        fast = U <= kUMax;
        if (fast) {
            // pad to a multiple of four with keys above every row, then
            // count in 16-byte broadcast reads
            if (tid < 4 && U + tid < kSortCap) ul[U + tid] = INT_MAX;
            lds_barrier();
            const int u4 = (U + 3) / 4;
            const int4* ul4 = reinterpret_cast<const int4*>(ul);
            for (int i = tid; i < U; i += NT) {
                const int32_t key = ul[i];
                int rank = 0;
#pragma unroll 4
                for (int j = 0; j < u4; ++j) {
                    const int4 v = ul4[j];
                    rank += (v.x < key) + (v.y < key) + (v.z < key) + (v.w < key);
                }
                L.urow[rank] = key;  // distinct keys: the ranks are a permutation of [0, U)
                ht[us[i]] = ((unsigned long long)rank << 32) | (uint32_t)key;
            }
            lds_barrier();
#pragma unroll
            for (int k = 0; k < EPT; ++k) {
                const int e = tid + k * NT;
                if (e < NQ) {
                    int32_t out = U;  // the zero row
                    if (ent[k] >= 0) {
                        // present: no insert stopped early when U <= kUMax
                        uint32_t h = hash(ent[k]);
                        unsigned long long v = ht[h];
                        for (int probe = 1; probe < kHashSlots && (uint32_t)v != (uint32_t)ent[k]; ++probe) {
                            h = (h + 1) & (kHashSlots - 1);
                            v = ht[h];
                        }
                        out = (uint32_t)v == (uint32_t)ent[k] ? (int32_t)(v >> 32) : U;
                    }
                    ent[k] = GEO::key(out);  // the entry's slot key (placed below)
                }
            }
            for (int r = tid; r < TM; r += NT) L.sidx[NTAPS * TM + r] = (uint16_t)GEO::key(U);
        }
    } else {
      // ranks of a W-word bitmap: thread tid owns words WPT*tid .. WPT*tid + WPT - 1
      auto bitmap_union = [&](auto words_const) __attribute__((always_inline)) {
        constexpr int W = decltype(words_const)::value;
        constexpr int WPT = W / NT;
        int32_t* wbase = reinterpret_cast<int32_t*>(L.scratch) + W;
        uint32_t wv[WPT];
        int cnt = 0;
#pragma unroll
        for (int w = 0; w < WPT; ++w) {
            wv[w] = bm[WPT * tid + w];
            cnt += __popc(wv[w]);
        }
        int incl = cnt;
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off);
            if (lane >= off) incl += v;
        }
        if (lane == 63) L.wsum[wave] = incl;
        lds_barrier();
        int base = incl - cnt;
        U = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            if (w < wave) base += L.wsum[w];
            U += L.wsum[w];
        }
        fast = U <= kUMax;
        {
            int b = base;
#pragma unroll
            for (int w = 0; w < WPT; ++w) {
                wbase[WPT * tid + w] = b;
                b += __popc(wv[w]);
            }
        }
        lds_barrier();
        if (fast) {
#pragma unroll
            for (int k = 0; k < EPT; ++k) {
                const int e = tid + k * NT;
                if (e < NQ) {
                    int32_t out = U;  // the zero row
                    if (ent[k] >= 0) {
                        const int32_t off = ent[k] - lo;
                        const int wi = off >> 5;
                        out = wbase[wi] + __popc(bm[wi] & ((1u << (off & 31)) - 1u));
                        // the union row at its rank: every union row is some
                        // entry's source, and entries sharing a source write
                        // the same value (a per-word walk of the set bits
                        // left most lanes idle behind the densest words:
                        // 6.6 of a 256^3-level tile's 19 us)
                        L.urow[out] = ent[k];
                    }
                    ent[k] = GEO::key(out);  // the entry's slot key (placed below)
                }
            }
            for (int r = tid; r < TM; r += NT) L.sidx[NTAPS * TM + r] = (uint16_t)GEO::key(U);
        }
      };
      if (wide) bitmap_union(std::integral_constant<int, kWinWordsWide>{});
      else bitmap_union(std::integral_constant<int, kWinWords>{});
    }
    if (fast) {
        // The slot keys go to their rows through a contiguous staging pass:
        // entry e = r NTAPS + o leaves a thread's registers for stg[e], then
        // each (tap, row) is read across and placed.  Stored straight from
        // the entry order, a wave's 64 lanes wrote TM x 2 bytes apart per tap,
        // into a few LDS banks (the plan of the 1,393,024-row 256^3 level:
        // 10.8 of a tile's 19 us).
        static_assert(NQ * 2 <= kSetupScratchWords * 4, "slot-key staging fits the scratch");
        lds_barrier();  // every thread is done with the bitmap / hash
        uint16_t* stg = reinterpret_cast<uint16_t*>(L.scratch);
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const int e = tid + k * NT;
            if (e < NQ) stg[e] = (uint16_t)ent[k];
        }
        lds_barrier();
        for (int q = tid; q < NQ; q += NT) {
            const int o = q / TM;
            const int r = q - o * TM;
            L.sidx[o * TM + slot_pos(r)] = stg[r * NTAPS + o];
        }
    }
    if (tid == 0) {
        // the active taps in ascending order, four per word; padding 0xff
        uint32_t m = (uint32_t)L.misc[0];
        for (int w = 0; w < kTapWords; ++w) {
            uint32_t word = 0;
            for (int b = 0; b < PD; ++b) {
                uint32_t t = 0xffu;
                if (m) {
                    t = (uint32_t)(__ffs(m) - 1);
                    m &= m - 1;
                }
                word |= t << (8 * b);
            }
            L.tlw[w] = word;
        }
        L.misc[3] = U;
        L.misc[4] = fast ? 1 : 0;
    }
    lds_barrier();
}

// One block per row tile of geometry GEO: runs the tile setup once and
// stores it, so every conv over the same index table skips it.
template <int NTAPS, typename GEO>
__global__ __launch_bounds__(512) void conv_plan_kernel(ConvArgs a, char* plan) {
    constexpr int TM = GEO::TM;
    __shared__ __attribute__((aligned(16))) uint32_t scratch[kSetupScratchWords];
    __shared__ __attribute__((aligned(16))) uint16_t sidx[(NTAPS + 1) * TM];
    __shared__ __attribute__((aligned(16))) uint32_t tlw[kTapWords];
    __shared__ __attribute__((aligned(16))) int32_t urow[GEO::UROWCAP];
    __shared__ __attribute__((aligned(16))) int32_t srow[TM];
    __shared__ int32_t wsum[8];
    __shared__ int32_t misc[8];
    const TileLds L{scratch, sidx, tlw, urow, srow, wsum, misc};
    const int64_t tm = blockIdx.x;
    tile_setup<NTAPS, 512, 4, GEO>(a, tm * TM, L);
    char* pt = plan + tm * GEO::plan_tile_bytes(NTAPS);
    int32_t* hdr = reinterpret_cast<int32_t*>(pt);
    const int U = misc[3];
    const int tid = threadIdx.x;
    if (tid < 8)
        hdr[tid] = tid == 0 ? U : tid == 1 ? misc[0] : tid == 2 ? misc[4] : tid == 3 ? kPlanMagic : 0;
    else if (tid < 16) hdr[tid] = (int32_t)tlw[tid - 8];
    for (int i = tid; i < TM; i += 512) reinterpret_cast<int32_t*>(pt + GEO::PLAN_SROW)[i] = srow[i];
    if (misc[4]) {
        for (int i = tid; i < U; i += 512)
            reinterpret_cast<int32_t*>(pt + GEO::PLAN_UROW)[i] = urow[i];
        for (int i = tid; i < (NTAPS + 1) * TM; i += 512)
            reinterpret_cast<uint16_t*>(pt + GEO::PLAN_SIDX)[i] = sidx[i];
    }
}

// Workgroups per CU a geometry is built for: GeoWide and GeoQuad fill the
// CU's LDS with one; GeoSmall's ~42 KB and GeoTall's ~53 KB admit three (register
// budget 168 per wave), two for 128-column tiles, whose 64 x 64 wave tiles
// need ~226 registers.
template <typename GEO, int TN>
constexpr int geo_blocks_per_cu() { return GEO::NBUF == 1 ? (TN >= 128 ? 2 : 3) : 1; }

// Whether a tile of TN columns can run the LayerNorm -> modulation -> SiLU
// epilogue: whole rows of at most 128 channels, and half the tile's rows in
// F32 inside the A area.  launch_conv refuses the norm epilogue where this
// is false, so no instantiation stores un-normalised rows.
template <typename GEO, int TN>
constexpr bool norm_epilogue_fits() {
    return TN <= 128 && GEO::TM / 2 * (TN + 4) * 4 <= GEO::NBUF * GEO::STAGE * 16;
}

template <typename T, bool Q8, bool PACKED, int NTAPS, int TN, int WM, int WN, int PD, typename GEO>
__global__ __launch_bounds__(WM * WN * 64, (geo_blocks_per_cu<GEO, TN>())) void conv_kernel(ConvArgs a) {
    using M = Mfma<T>;
    using P = Panel<T, Q8>;
    constexpr int TM = GEO::TM;
    constexpr int NW = WM * WN;
    constexpr int NT = NW * 64;
    constexpr int ES = sizeof(T);
    constexpr int KC = P::KC;
    constexpr int WTM = TM / WM;
    constexpr int WTN = TN / WN;
    constexpr int BR = M::BR;                   // output rows per MFMA block
    constexpr int BC = M::BC;                   // output channels per MFMA block
    constexpr int NH = P::NH;                   // channel blocks per 32-channel panel
    constexpr int FM = WTM / BR;                // the wave's row blocks
    constexpr int FC = WTN / BC;                // the wave's channel blocks
    // Weight loads: packed 16-bit weights per 16-channel block (a panel's
    // word h is its block h, so a wave's width need only be a multiple of
    // 16: the 96-column tiles' 48-channel waves), the other layouts per
    // 32-channel panel of P::NG words.
    constexpr bool BLK = PACKED && !Q8 && P::G == 1 && P::NG == NH && P::KS == 1;
    constexpr int LG = BLK ? FC : WTN / 32;     // load groups per step
    constexpr int LW = BLK ? 1 : P::NG;         // words per load group
    constexpr int NQ = NTAPS * TM;
    constexpr int STAGE = GEO::STAGE;           // 16-byte units per A buffer
    constexpr int NBUF = GEO::NBUF;             // A buffers
    constexpr int ABYTES = NBUF * STAGE * 16;   // the A area (reused by the setup and epilogue)
    constexpr int NPART = 4;                    // parts of a chunk's staging
    static_assert(FM >= 1 && FC >= 1 && FM * BR == WTM && FC * BC == WTN && (BLK || WTN % 32 == 0) &&
                      WTM * WM == TM && WTN * WN == TN,
                  "wave geometry");
    static_assert(!Q8 || ES == 2, "Q8_0 weights feed 16-bit MFMA operands");
    static_assert(NTAPS <= 32, "tap mask is 32-bit");
    static_assert(kSetupScratchWords * 4 <= ABYTES, "setup scratch aliases the A stage");
    static_assert(PD == 4, "the step groups pack four taps per word");
    static_assert(NBUF == 1 || NBUF == 2 || NBUF == 4, "one, two or four A buffers");

    __shared__ u32x4 Au[NBUF * STAGE];  // A buffers: (U + 1) rows x 64 bytes each
    __shared__ __attribute__((aligned(16))) uint16_t sidx[NQ + TM];  // slot keys; row NTAPS = zeros
    __shared__ __attribute__((aligned(16))) uint32_t tlw[kTapWords]; // step taps, 4 per word
    __shared__ __attribute__((aligned(16))) int32_t urow[GEO::UROWCAP];  // source row of each union slot
    __shared__ __attribute__((aligned(16))) int32_t srow[TM];        // output row of each tile row
    __shared__ int32_t wsum[NW];
    __shared__ __attribute__((aligned(16))) int32_t misc[8];
    __shared__ __attribute__((aligned(16))) float sbias[TN];
    // Per-wave epilogue (16-bit outputs of 8-wave tiles): once a wave is done
    // with the last chunk it writes its own block through a private LDS
    // region and stores it, while the other waves still compute.  The
    // regions are the stage buffer the last chunk does not read (two
    // buffers), and PWX more here for the waves it cannot hold (all of them
    // with four buffers, whose waves run a group's chunks without barriers).
    constexpr int PW_PITCH = WTN * ES + 16;      // bytes per row of a wave's block
    constexpr int PW_BYTES = WTM * PW_PITCH;
    constexpr bool PWE = ES == 2 && (NBUF == 2 || NBUF == 4) && NW == 8 && WTM * WTN <= 4096;
    constexpr int PW_IN_STAGE = PWE && NBUF == 2 ? STAGE * 16 / PW_BYTES : 0;  // regions in the free buffer
    constexpr int PWX = PWE && PW_IN_STAGE < NW ? NW - PW_IN_STAGE : 0;
    __shared__ __attribute__((aligned(16))) char pw_extra[PWX > 0 ? PWX * PW_BYTES : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform

    // Tile mapping: the tiles of the full row tiles XCD-major (workgroup b
    // runs on XCD b % 8, each XCD gets a contiguous range of them), then the
    // tiles of a partial last row tile, which run last and cost little.
    // Within the range, row tile by row tile (the column tiles of a row
    // tile share its gathered rows in the XCD's L2), or, with weights larger
    // than half an L2 (col_major), column tile by column tile: the tiles an
    // XCD runs at once then share their weight panels (SubM 128 -> 1024 and
    // 1024 -> 1024 over 11,774 rows, Q8_0 C = 768: 3-4 % faster).
    int64_t tile;
    const int64_t hb = a.tiles_per_xcd * 8;  // workgroups of the XCD-major part
    if ((int64_t)blockIdx.x < hb) {
        const int64_t xcd = blockIdx.x & 7;
        const int64_t local = blockIdx.x >> 3;
        tile = xcd * a.tiles_per_xcd + local;
        if (tile >= a.heavy_tiles) return;
    } else {
        tile = a.heavy_tiles + ((int64_t)blockIdx.x - hb);
        if (tile >= a.total_tiles) return;
    }
    int64_t tm;
    int tn;
    if (tile < a.heavy_tiles && a.col_major) {
        const int64_t mfull = a.heavy_tiles / a.tiles_n;  // full row tiles
        tm = tile % mfull;
        tn = (int)(tile / mfull);
    } else {
        tm = tile / a.tiles_n;
        tn = (int)(tile % a.tiles_n);
    }
    const int64_t r0 = tm * TM;
    const int co0 = tn * TN;

    for (int c = tid; c < TN; c += NT) sbias[c] = a.bias ? M::ld(a.bias, co0 + c) : 0.0f;

    // a self-refreshing plan tile over changed rows is not read
    bool dirty = false;
    if (a.plan_dirty) {
        const int64_t f0 = r0 / 128, nf = (a.n_out + 127) / 128;
        for (int64_t f = f0; f < nf && f * 128 < r0 + TM; ++f)
            for (int o = 0; o < NTAPS; ++o) dirty |= a.plan_dirty[f * NTAPS + o] != 0;
    }

    uint32_t tile_mask;
    int U;
    bool fast;
    bool planned = false;
    if (a.plan) {
        // the tile's setup from the plan: one batch of 16-byte copies of the
        // whole plan tile (header, tap words, output rows, union rows, slot
        // keys -- contiguous in the plan) into LDS, all loads in flight at once
        const u32x4* pt = reinterpret_cast<const u32x4*>(static_cast<const char*>(a.plan) +
                                                         tm * GEO::plan_tile_bytes(NTAPS));
        constexpr int NHD = 2, NTW = 2;              // header and tap-word units
        constexpr int NSR = TM / 4;                  // srow units
        constexpr int NUR = GEO::UROWCAP / 4;        // urow units (the stage's union capacity)
        constexpr int NURP = GEO::PUROWCAP / 4;      // urow units in the plan
        constexpr int NSI = (NTAPS + 1) * TM / 8;    // sidx units
        constexpr int TOTAL = NHD + NTW + NSR + NUR + NSI;
        constexpr int IT = (TOTAL + NT - 1) / NT;
        static_assert(GEO::PLAN_SROW == 16 * (NHD + NTW) && GEO::PLAN_UROW == GEO::PLAN_SROW + 16 * NSR &&
                          GEO::PLAN_SIDX == GEO::PLAN_UROW + 16 * NURP && NURP >= NUR,
                      "plan sections are contiguous");
        u32x4 pv[IT];
#pragma unroll
        for (int k = 0; k < IT; ++k) {
            const int u = tid + k * NT;
            // union rows past the stage's capacity are not copied: such a
            // tile takes the fallback, which does not read them
            if (u < TOTAL) pv[k] = pt[u < NHD + NTW + NSR + NUR ? u : u + (NURP - NUR)];
        }
#pragma unroll
        for (int k = 0; k < IT; ++k) {
            const int u = tid + k * NT;
            if (u >= TOTAL) continue;
            u32x4* dst;
            if (u < NHD) dst = reinterpret_cast<u32x4*>(misc) + u;
            else if (u < NHD + NTW) dst = reinterpret_cast<u32x4*>(tlw) + (u - NHD);
            else if (u < NHD + NTW + NSR) dst = reinterpret_cast<u32x4*>(srow) + (u - NHD - NTW);
            else if (u < NHD + NTW + NSR + NUR) dst = reinterpret_cast<u32x4*>(urow) + (u - NHD - NTW - NSR);
            else dst = reinterpret_cast<u32x4*>(sidx) + (u - NHD - NTW - NSR - NUR);
            *dst = pv[k];
        }
        lds_barrier();
        // a tile of a section the plan's builder skipped has no marker: set it up here
        planned = misc[3] == kPlanMagic && !dirty;
        U = misc[0];
        tile_mask = (uint32_t)misc[1];
        fast = misc[2] != 0;
    }
    if constexpr (NTAPS == 1) {
        if (!planned && a.idx == nullptr && a.row_perm == nullptr && a.class_rows == 0) {
            // the dense 1x1x1 conv (identity map): the tile's union is its own
            // rows in order, each row's slot its own -- no deduplication (the
            // general setup cost such a tile more than its one-tap loop)
            const int nr = (int)min<int64_t>(TM, a.n_out - r0);
            for (int r = tid; r < TM; r += NT) {
                srow[r] = r < nr ? (int32_t)(r0 + r) : -1;
                urow[r] = (int32_t)(r0 + r);
                sidx[slot_pos(r)] = (uint16_t)GEO::key(r < nr ? r : nr);
                sidx[TM + r] = (uint16_t)GEO::key(nr);
            }
            if (tid < kTapWords) tlw[tid] = tid == 0 ? 0xffffff00u : 0xffffffffu;  // tap 0, then padding
            lds_barrier();
            U = nr;
            tile_mask = 1u;
            fast = true;
            planned = true;
        }
    }
    if (!planned) {
        // tile_setup writes misc[3] only after its first barriers, once every
        // thread has read the marker above
        const TileLds L{reinterpret_cast<uint32_t*>(Au), sidx, tlw, urow, srow, wsum, misc};
        tile_setup<NTAPS, NT, PD, GEO>(a, r0, L);
        tile_mask = (uint32_t)misc[0];
        U = misc[3];
        fast = misc[4] != 0;
        if (a.idx_cache && dirty && tn == 0) {
            // refresh: this tile's plan tile (as conv_plan_kernel writes it)
            // and its cached index entries.  No workgroup of this launch reads
            // them: every tile over these rows is flagged.
            char* pt = const_cast<char*>(static_cast<const char*>(a.plan)) +
                       tm * GEO::plan_tile_bytes(NTAPS);
            int32_t* hdr = reinterpret_cast<int32_t*>(pt);
            if (tid < 8)
                hdr[tid] = tid == 0 ? U : tid == 1 ? (int32_t)tile_mask : tid == 2 ? (int32_t)fast
                         : tid == 3 ? (int32_t)kPlanMagic : 0;
            else if (tid < 16) hdr[tid] = (int32_t)tlw[tid - 8];
            for (int i = tid; i < TM; i += NT) reinterpret_cast<int32_t*>(pt + GEO::PLAN_SROW)[i] = srow[i];
            if (fast) {
                for (int i = tid; i < U; i += NT) reinterpret_cast<int32_t*>(pt + GEO::PLAN_UROW)[i] = urow[i];
                for (int i = tid; i < (NTAPS + 1) * TM; i += NT)
                    reinterpret_cast<uint16_t*>(pt + GEO::PLAN_SIDX)[i] = sidx[i];
            }
            for (int q = tid; q < NTAPS * TM; q += NT) {
                const int o = q / TM;
                const int64_t rr = r0 + (q - o * TM);
                if (rr >= a.n_out) continue;
                const int64_t e = a.idx_layout == SPC_IDX_TOKEN_MAJOR ? rr * NTAPS + o
                                                                     : (int64_t)o * a.n_out + rr;
                a.idx_cache[e] = a.idx[e];
            }
        }
    }
    // tile-uniform values: keep them (and the control flow they drive) scalar
    U = __builtin_amdgcn_readfirstlane(U);
    tile_mask = (uint32_t)__builtin_amdgcn_readfirstlane(tile_mask);
    fast = __builtin_amdgcn_readfirstlane((int)fast) != 0;

    // source row of (tap o, tile row r), -1 when missing (fallback tiles)
    auto src_of = [&](int o, int r) __attribute__((always_inline)) -> int32_t {
        const int32_t t = srow[r];
        if (t < 0) return -1;
        int32_t s;
        if (NTAPS == 1 && a.idx == nullptr) s = t;  // identity map (dense 1x1x1 conv)
        else if (a.idx_layout == SPC_IDX_TOKEN_MAJOR) s = a.idx[(int64_t)t * NTAPS + o];
        else s = a.idx[(int64_t)o * a.n_out + t];
        return (s < 0 || s >= a.n_in) ? -1 : s;
    };

    const int nt = __popc(tile_mask);
    const int kch = a.cin / KC;
    const int ncol32 = a.cout / 32;

    const int wm = wave / WN;
    const int wn = wave % WN;

    // accumulators start at the bias: element 4g + e of lane l holds output
    // channel M::run(l, g) + e of its channel block
    typename M::acc_t acc[FM][FC];
#pragma unroll
    for (int c = 0; c < FC; ++c) {
        floatx4 b4[M::NRUN];
#pragma unroll
        for (int g = 0; g < M::NRUN; ++g)
            b4[g] = *reinterpret_cast<const floatx4*>(sbias + wn * WTN + c * BC + M::run(lane, g));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int k = 0; k < 4 * M::NRUN; ++k) acc[i][c][k] = b4[k / 4][k % 4];
    }

    const char* xb = static_cast<const char*>(a.x);
    const u32x4 zero4 = {0u, 0u, 0u, 0u};

    struct Slot {
        u32x4 q[LG][LW];
        float d[Q8 ? FC : 1];  // Q8_0: scale of the lane's channel in block j NH + h
    };

    // Packed weights through a buffer resource: the panel offset is a scalar,
    // the lane offset a constant register, so a fragment load costs no vector
    // address arithmetic (and reads past the packed size return zeros).
    const uint32_t wbytes =
        (uint32_t)((int64_t)a.ntaps * max(1, a.n_classes) * a.cin * a.cout * P::WB);
    // weight class of the tile: its first packed tap (class_rows is a multiple of the tile height)
    const uint32_t wtap0 = a.class_rows > 0 ? (uint32_t)(r0 / a.class_rows) * NTAPS : 0u;
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.w), (short)0, (int)wbytes, 0x00020000);
    // weight operands of (tap o, chunk kc) for this wave's LG load groups
    auto load_b = [&](int o, int kc, Slot& sl) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < LG; ++j) {
            const int c32 = (co0 + wn * WTN) / 32 + j;  // wave-uniform (panel groups)
            if constexpr (BLK) {
                const int cb = (co0 + wn * WTN) / BC + j;  // 16-channel block, wave-uniform
                const uint32_t panel = ((wtap0 + (uint32_t)o) * (uint32_t)kch + (uint32_t)kc) *
                                           (uint32_t)ncol32 + (uint32_t)(cb / NH);
                const int poff = (int)(panel * (uint32_t)(P::NG * 1024) + (uint32_t)(cb % NH) * 1024u);
                sl.q[j][0] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, lane * 16, poff, 0));
            } else if constexpr (PACKED) {
                const uint32_t panel =
                    ((wtap0 + (uint32_t)o) * (uint32_t)kch + (uint32_t)kc) * (uint32_t)ncol32 + (uint32_t)c32;
                const int poff = (int)(panel * (uint32_t)(P::NG * 1024));
#pragma unroll
                for (int g = 0; g < P::NG; ++g)
                    sl.q[j][g] = __builtin_bit_cast(
                        u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, lane * 16 + g * 1024, poff, 0));
                if constexpr (Q8) {
#pragma unroll
                    for (int h = 0; h < NH; ++h)
                        sl.d[j * NH + h] = static_cast<const float*>(
                            a.wscale)[((int64_t)o * kch + kc) * a.cout + c32 * 32 + P::co_of(h, lane)];
                }
            } else {
                // [cout, ntaps, cin]: fragment f of word g from its own row
#pragma unroll
                for (int g = 0; g < P::NG; ++g) {
                    uint32_t words[4];
                    constexpr int WPF = 4 / P::G;  // 32-bit words per fragment
#pragma unroll
                    for (int i = 0; i < P::G; ++i) {
                        const int f = g * P::G + i;
                        const int64_t co = c32 * 32 + P::co_of(f, lane);
                        const int64_t el = (co * NTAPS + o) * a.cin + (int64_t)kc * KC + P::ci_of(f, lane);
                        const uint32_t* wp = reinterpret_cast<const uint32_t*>(
                            static_cast<const char*>(a.w) + el * P::WB);
#pragma unroll
                        for (int h = 0; h < WPF; ++h) words[i * WPF + h] = wp[h];
                    }
                    sl.q[j][g] = u32x4{words[0], words[1], words[2], words[3]};
                }
                if constexpr (Q8) {
#pragma unroll
                    for (int h = 0; h < NH; ++h) {
                        const int64_t co = c32 * 32 + P::co_of(h, lane);
                        const int64_t el = (co * NTAPS + o) * a.cin + (int64_t)kc * KC;
                        sl.d[j * NH + h] = f16_bits_to_f32(static_cast<const uint16_t*>(a.wscale)[el >> 5]);
                    }
                }
            }
        }
    };

    // weight fragment f (k-step f / NH, channel block f % NH) of panel j from a loaded slot
    auto b_frag = [&](const Slot& sl, int j, int f) __attribute__((always_inline)) {
        typename M::frag fr;
        const u32x4 wv4 = sl.q[j][f / P::G];
        if constexpr (Q8) {
            // 8 int8 quants of this fragment -> bf16(d * q)
            fr = q8_dequant8((f % P::G) == 0 ? wv4.x : wv4.z, (f % P::G) == 0 ? wv4.y : wv4.w,
                             sl.d[j * NH + f % NH]);
        } else if constexpr (P::G == 1) {
            fr = __builtin_bit_cast(typename M::frag, wv4);
        } else {
            // explicit component select: indexing the vector by (f % G) read
            // component 0 for every k-step in generated code
            const int c = f % P::G;
            const uint32_t word = c == 0 ? wv4.x : c == 1 ? wv4.y : c == 2 ? wv4.z : wv4.w;
            fr = __builtin_bit_cast(float, word);
        }
        return fr;
    };

    typedef typename M::frag AFrag[P::KS][FM];
    // The MFMA computes the transposed block (weights as the row operand,
    // gathered features as the column one): the accumulator of lane l then
    // holds output row l % BR and four consecutive output channels from
    // M::run(l, g) per run g, stored straight to global memory.
    // fa_const: the wave's live row blocks (FM, or fewer in a partial last
    // row tile, whose dead blocks are skipped)
    auto mma_step = [&](const AFrag& af, const Slot& bs, auto fa_const) __attribute__((always_inline)) {
        constexpr int FA = decltype(fa_const)::value;
        if constexpr (BLK) {
#pragma unroll
            for (int c = 0; c < FC; ++c) {
                const typename M::frag bf = __builtin_bit_cast(typename M::frag, bs.q[c][0]);
#pragma unroll
                for (int i = 0; i < FA; ++i) acc[i][c] = M::mma(bf, af[0][i], acc[i][c]);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < P::KS; ++ks) {
#pragma unroll
                for (int j = 0; j < LG; ++j) {
#pragma unroll
                    for (int h = 0; h < NH; ++h) {
                        const typename M::frag bf = b_frag(bs, j, ks * NH + h);
#pragma unroll
                        for (int i = 0; i < FA; ++i)
                            acc[i][j * NH + h] = M::mma(bf, af[ks][i], acc[i][j * NH + h]);
                    }
                }
            }
        }
    };
    // A fragments of k-slices of BR rows per row block.  sl[] holds slot
    // keys; the byte of each k-step within the 64-byte row is a lane
    // constant, its segment placed by the geometry's row layout.
    auto read_frags = [&](int buf, const int* sl, AFrag& f, auto fa_const) __attribute__((always_inline)) {
        constexpr int FA = decltype(fa_const)::value;
        const char* ab = reinterpret_cast<const char*>(Au + buf * STAGE);
#pragma unroll
        for (int ks = 0; ks < P::KS; ++ks) {
            const int byte = (ks * M::KSUB + (lane / BR) * M::EPL) * ES;  // within the 64-byte row
#pragma unroll
            for (int i = 0; i < FA; ++i)
                f[ks][i] = *reinterpret_cast<const typename M::frag*>(
                    ab + GEO::unit(sl[i], byte >> 4) * 16 + (byte & 15));
        }
    };
    // union slots of the wave's rows for sidx row `row` (a tap, or NTAPS =
    // zeros): 16-row blocks read four keys (a 64-row wave tile) or two (32
    // rows) at once from the interleaved layout
    auto read_slots = [&](int row, int* sl, auto fa_const) __attribute__((always_inline)) {
        constexpr int FA = decltype(fa_const)::value;
        const uint16_t* st = sidx + row * TM;
        if constexpr (BR == 16 && WTM % 64 == 0) {
#pragma unroll
            for (int q = 0; q < (FA + 3) / 4; ++q) {
                const u32x2 v = *reinterpret_cast<const u32x2*>(st + wm * WTM + 64 * q + 4 * (lane & 15));
#pragma unroll
                for (int i = 0; i < 4 && 4 * q + i < FA; ++i)
                    sl[4 * q + i] = (int)((i & 1) ? v[i >> 1] >> 16 : v[i >> 1] & 0xffffu);
            }
        } else if constexpr (BR == 16 && WTM == 32) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(
                st + (wm * WTM & ~63) + 4 * (lane & 15) + ((wm * WTM >> 4) & 3));
            sl[0] = (int)(v & 0xffffu);
            if constexpr (FA > 1) sl[1] = (int)(v >> 16);
        } else {
#pragma unroll
            for (int i = 0; i < FA; ++i) sl[i] = st[slot_pos(wm * WTM + i * BR + (lane % BR))];
        }
    };
    const auto fm_all = std::integral_constant<int, FM>{};

    // The fast path stages through LDS DMA with 32-bit offsets from the
    // tile's lowest source row.
    const int64_t rowbytes = (int64_t)a.cin * ES;
    const bool dma = fast && nt > 0 && U > 0 && U <= GEO::UMAX &&
                     (int64_t)(urow[U - 1] - urow[0] + 1) * rowbytes <= 0x7fffffffLL;

    if (dma) {
        // ---- A staging through LDS DMA -----------------------------------
        // A chunk's stage is U + 1 rows in the geometry's row layout, in
        // 64-unit blocks of 16 bytes; one buffer_load_dwordx4 ... lds fills a
        // block (lane l -> unit 64 * block + l).  A unit holds one segment of
        // one union row; padding units (the 80-byte layout's fifth unit), the
        // zero row U and units past it read out of range, which writes zeros.  The next chunk's blocks
        // are issued in NPART parts at the starts of the first step groups;
        // they land in the free buffer while the MFMAs run and are waited
        // for once, before the chunk barrier.
        const int32_t row0 = __builtin_amdgcn_readfirstlane(urow[0]);
        const uint32_t nrec = (uint32_t)min<int64_t>((a.n_in - row0) * rowbytes, 0x7fffffffLL);
        const uint64_t xbase = reinterpret_cast<uint64_t>(xb + (int64_t)row0 * rowbytes);
        // buffer descriptor: base, stride 0, num_records, raw-buffer flags
        const u32x4 xrsrc = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)xbase),
                             (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(xbase >> 32) & 0xffffu),
                             (uint32_t)__builtin_amdgcn_readfirstlane(nrec), 0x00020000u};
        const uint32_t au_lds = __builtin_amdgcn_readfirstlane(
            (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) u32x4*)Au));
        const int nblk = ((U + 1) * GEO::PITCH + 63) / 64;
        // Wave w fills blocks w + NW j.  The per-lane source offsets do not
        // depend on the chunk (it enters as the scalar offset), so they are
        // computed once per tile and kept in registers.
        constexpr int NJ = (STAGE / 64 + NW - 1) / NW;  // blocks per wave, at most
        uint32_t doff[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int v = (wave + NW * j) * 64 + lane;
            const int r = v / GEO::PITCH;
            const int sg = GEO::SW ? (v & 3) ^ GEO::swz(r) : v - r * GEO::PITCH;
            doff[j] = 0x80000000u;  // out of range: zeros
            if (sg < kSegs && r < U)
                doff[j] = (uint32_t)(urow[r] - row0) * (uint32_t)rowbytes + (uint32_t)(sg * 16);
        }
        // part h of a chunk: the wave's blocks j in [h NJ / NPART, (h + 1) NJ / NPART)
        auto stage_part = [&](int kc, int buf, auto h_const) __attribute__((always_inline)) {
            constexpr int H = decltype(h_const)::value;
            const uint32_t koff = (uint32_t)__builtin_amdgcn_readfirstlane(kc * KC * ES);
#pragma unroll
            for (int j = H * NJ / NPART; j < (H + 1) * NJ / NPART; ++j) {
                const int blk = wave + NW * j;
                if (blk < nblk) lds_dma_x4(xrsrc, au_lds + (uint32_t)((buf * STAGE + blk * 64) * 16), doff[j], koff);
            }
        };
        // part h for a run-time h < NPART
        auto stage_part_rt = [&](int kc, int buf, int h) __attribute__((always_inline)) {
            static_assert(NPART == 4, "parts");
            if (h == 0) stage_part(kc, buf, std::integral_constant<int, 0>{});
            else if (h == 1) stage_part(kc, buf, std::integral_constant<int, 1>{});
            else if (h == 2) stage_part(kc, buf, std::integral_constant<int, 2>{});
            else stage_part(kc, buf, std::integral_constant<int, 3>{});
        };
        // four buffers: the chunks g0 .. g0 + 3 at once, chunk c in buffer c % 4
        // (one staging latency per four chunks instead of one per chunk)
        auto stage_group = [&](int g0) __attribute__((always_inline)) {
            for (int c = g0; c < kch && c < g0 + NBUF; ++c)
                for (int h = 0; h < NPART; ++h) stage_part_rt(c, c % NBUF, h);
        };
        // vector-memory loads per step (weight words, plus Q8_0 scales)
        constexpr int LPS = PACKED ? LG * LW + (Q8 ? FC : 0) : 0;
        // Four buffers with at most two step groups per chunk (the stride-2
        // taps): a whole-chunk weight ring.  Every step's weights are loaded
        // one chunk ahead and each chunk is staged at the start of the one
        // before it, so that staging has a chunk's compute to land: loads
        // complete in issue order, and the first weight load queued behind
        // it is needed only in its own chunk.  Chunks 0 and 1 are staged
        // together; chunk 0 alone is waited for.
        constexpr bool DR = NBUF == 4 && NTAPS <= 2 * PD && PACKED;
        constexpr int RS = DR ? 2 * PD : PD;  // weight ring slots
        static_assert(!DR || (2 * PD * LPS < 64 && NJ < 64), "vmcnt range");
        const int njw = wave < nblk ? min(NJ, (nblk - wave + NW - 1) / NW) : 0;  // this wave's blocks per chunk
        auto stage_chunk = [&](int kc) __attribute__((always_inline)) {
            for (int h = 0; h < NPART; ++h) stage_part_rt(kc, kc % NBUF, h);
        };

        // Steps of a chunk: the active taps in ascending order, padded to a
        // multiple of PD with steps that read the zero slot (row NTAPS)
        // against the first tap's weights.  A group of PD steps is unrolled;
        // every register-array index inside it is a compile-time constant:
        // B operands of step i live in ring[i % PD] (loaded PD steps ahead;
        // the whole-chunk ring: ring[i], loaded a chunk ahead),
        // A fragments in afr[i % 2] (read one step ahead, within a chunk),
        // union slots in sreg[i % 2] (read two steps ahead; slots do not
        // depend on the chunk, so they run ahead across chunk boundaries).
        // (whole-chunk ring: always two groups, the second possibly all padding)
        const int ngr = DR ? 2 : (nt + PD - 1) / PD;
        const int tfirst = __ffs(tile_mask) - 1;
        auto b_tap = [&](uint32_t word, int b) __attribute__((always_inline)) -> int {
            const int t = (int)((word >> (8 * b)) & 0xffu);
            return t == 0xff ? tfirst : t;
        };
        auto s_row = [&](uint32_t word, int b) __attribute__((always_inline)) -> int {
            const int t = (int)((word >> (8 * b)) & 0xffu);
            return t == 0xff ? NTAPS : t;
        };

        // A wave none of whose rows exists (the partial last row tile) only
        // does its share of the staging and the barriers.
        int has_row = 0;
        for (int k = lane; k < WTM; k += 64) has_row |= srow[wm * WTM + k] >= 0;
        if (__builtin_amdgcn_ballot_w64(has_row != 0) == 0) {
            // the same barriers as the working waves, in the same order
            if constexpr (DR) {
                stage_chunk(0);
                if (kch > 1) stage_chunk(1);
                dma_barrier<0>();
                for (int kc = 1; kc < kch; ++kc) {
                    dma_barrier<0>();
                    if (kc + 1 < kch) stage_chunk(kc + 1);
                }
            } else if constexpr (NBUF == 4) {
                for (int g0 = 0; g0 < kch; g0 += NBUF) {
                    if (g0 > 0) lds_barrier();
                    stage_group(g0);
                    dma_barrier<0>();
                }
            } else {
                for (int h = 0; h < NPART; ++h) stage_part_rt(0, 0, h);
                dma_barrier<0>();
                for (int kc = 0; kc + 1 < kch; ++kc) {
                    if constexpr (NBUF == 1) lds_barrier();  // the buffer is free
                    for (int h = 0; h < NPART; ++h) stage_part_rt(kc + 1, NBUF == 1 ? 0 : (kc & 1) ^ 1, h);
                    dma_barrier<0>();
                }
            }
        } else {
          auto run_tile = [&](auto fa_const) __attribute__((always_inline)) {
            constexpr int FA = decltype(fa_const)::value;
            Slot ring[RS];
            AFrag afr[2];
            int sreg[2][FM];
            // the tap words in scalar registers: tw0 holds the running group's
            // word, the rest shift down one word per group; tw_first restores
            // them at every chunk start
            uint32_t tw_first[kTapWords], tw[kTapWords];
#pragma unroll
            for (int w = 0; w < kTapWords; ++w) tw_first[w] = __builtin_amdgcn_readfirstlane(tlw[w]);

            {
                const uint32_t w0 = tw_first[0];
#pragma unroll
                for (int p = 0; p < PD; ++p) load_b(b_tap(w0, p), 0, ring[p]);
                if constexpr (DR) {
                    const uint32_t w1f = tw_first[1];
#pragma unroll
                    for (int p = 0; p < PD; ++p) load_b(b_tap(w1f, p), 0, ring[PD + p]);
                }
                read_slots(s_row(w0, 0), sreg[0], fa_const);
                read_slots(s_row(w0, 1), sreg[1], fa_const);
                // (the weights go first: with the staging first, measured
                // 0.1-0.25 us later to the first step)
                if constexpr (DR) stage_chunk(0);
                else if constexpr (NBUF == 4) stage_group(0);
                else for (int h = 0; h < NPART; ++h) stage_part_rt(0, 0, h);
                if constexpr (DR) {
                    if (kch > 1) stage_chunk(1);
                    // chunk 0 and the ring have landed; this wave's loads of
                    // chunk 1 (the youngest) may still be in flight
                    dma_barrier_le<NJ>(kch > 1 ? njw : 0);
                } else {
                    dma_barrier<0>();
                }
                read_frags(0, sreg[0], afr[0], fa_const);
            }

            for (int kc = 0; kc < kch; ++kc) {
                const int buf = NBUF == 1 ? 0 : NBUF == 2 ? kc & 1 : kc % NBUF;
                // two buffers: the next chunk is staged while this one runs
                const bool more = NBUF == 2 && kc + 1 < kch;
                if (kc > 0) {
                    if constexpr (DR) {
                        // this chunk has landed: younger than its staging are
                        // exactly the last chunk's 2 PD steps of weight loads;
                        // then stage the next chunk (its buffer's chunk, three
                        // back, is done in every wave)
                        dma_barrier<2 * PD * LPS>();
                        if (kc + 1 < kch) stage_chunk(kc + 1);
                    } else if constexpr (NBUF == 4) {
                        // a group's first chunk: once every wave is done with
                        // the last group, stage this one and wait for it
                        if (kc % NBUF == 0) {
                            lds_barrier();
                            stage_group(kc);
                            dma_barrier<0>();
                        }
                    } else if constexpr (NBUF == 1) {
                        // one buffer: once every wave is done reading the last
                        // chunk (the barrier's fence waits for this wave's LDS
                        // reads), stage this one and wait for it; the weight
                        // prefetches of its first steps are older and land too
                        lds_barrier();
                        for (int h = 0; h < NPART; ++h) stage_part_rt(kc, 0, h);
                        dma_barrier<0>();
                    } else {
                        // chunk staged; every wave done with the other buffer.  With
                        // ngr >= NPART the last part preceded a whole group's loads.
                        if (ngr >= NPART && LPS > 0) dma_barrier<PD * LPS>();
                        else dma_barrier<0>();
                    }
                    read_frags(buf, sreg[0], afr[0], fa_const);
                }
#pragma unroll
                for (int w = 0; w < kTapWords; ++w) tw[w] = tw_first[w];
                // The last group of a chunk is peeled: its steps past the chunk's
                // taps (padding) skip their MFMAs but keep their loads, so every
                // step issues the same number of weight loads.
                const int nreal = nt - PD * (ngr - 1);  // real steps of the last group
                auto run_group = [&](int g, auto last_const) __attribute__((always_inline)) {
                    constexpr bool last_g = decltype(last_const)::value;
                    const uint32_t w0 = tw[0];
                    const uint32_t w1 = last_g ? tw_first[0] : tw[1];
                    // the loads: the steps PD ahead, or with the whole-chunk
                    // ring this group's steps of the next chunk
                    constexpr int RB = DR && last_g ? PD : 0;  // the group's ring slots
                    const uint32_t wl = DR ? w0 : w1;
                    const int kc_next = DR || last_g ? kc + 1 : kc;
                    const int kc_b = min(kc_next, kch - 1);  // past the last chunk: a valid, unused panel
                    if (more && g < NPART) stage_part_rt(kc + 1, buf ^ 1, g);
                    __builtin_amdgcn_sched_barrier(0);  // the part's loads precede the group's
                    auto step = [&](auto u_const) __attribute__((always_inline)) {
                        constexpr int u = decltype(u_const)::value;
                        // slots of the step after next (they do not depend on the chunk)
                        read_slots(u + 2 < PD ? s_row(w0, u + 2) : s_row(w1, u + 2 - PD), sreg[u & 1], fa_const);
                        // A fragments of the next step; after a chunk's last step they
                        // are re-read behind the barrier, so this read is unused
                        read_frags(buf, sreg[(u + 1) & 1], afr[(u + 1) & 1], fa_const);
                        if constexpr (last_g && (u > 0 || DR)) {
                            if (u < nreal) mma_step(afr[u & 1], ring[RB + u], fa_const);
                        } else {
                            mma_step(afr[u & 1], ring[RB + u], fa_const);
                        }
                        load_b(b_tap(wl, u), kc_b, ring[RB + u]);
                        // issue order: slot reads, then MFMAs interleaved with the
                        // fragment reads and their address arithmetic, then the
                        // weight loads
                        constexpr int NMF = P::KS * FA * FC;
                        constexpr int NFR = P::KS * FA;
                        __builtin_amdgcn_sched_group_barrier(0x100, FA, 0);
#pragma unroll
                        for (int q = 0; q < NMF; ++q) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            if (q < NFR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                            // Q8_0: room for the in-register dequantisation
                            __builtin_amdgcn_sched_group_barrier(0x002, Q8 ? 6 : 2, 0);
                        }
                        __builtin_amdgcn_sched_group_barrier(0x020, LG * LW, 0);
                        // nothing crosses a step boundary: without this fence the
                        // scheduler sinks every weight load of the group to its
                        // end, which leaves the next group's first steps waiting
                        __builtin_amdgcn_sched_barrier(0);
                    };
                    step(std::integral_constant<int, 0>{});
                    step(std::integral_constant<int, 1>{});
                    step(std::integral_constant<int, 2>{});
                    step(std::integral_constant<int, 3>{});
#pragma unroll
                    for (int w = 0; w + 1 < kTapWords; ++w) tw[w] = tw[w + 1];
                    // 8 waves: waves w and w + 4 share a SIMD, and the older
                    // one wins issue, so waves 4-7 fell ~3.4 us behind in
                    // every chunk and ended it alone; taking turns at the
                    // higher priority every step group keeps the pair
                    // together (C=128 over 4 ellipsoid shells, 62,710 rows:
                    // 55.3 -> 54.2 us)
                    if constexpr (NW == 8) {
                        if (((g + (wave >> 2)) & 1) != 0) __builtin_amdgcn_s_setprio(1);
                        else __builtin_amdgcn_s_setprio(0);
                    }
                };
                for (int g = 0; g + 1 < ngr; ++g) run_group(g, std::false_type{});
                run_group(ngr - 1, std::true_type{});
                if (more)  // short chunks: the parts the group loop did not reach
                    for (int h = ngr; h < NPART; ++h) stage_part_rt(kc + 1, buf ^ 1, h);
            }
          };
            // A wave of the partial last row tile whose rows end inside its
            // first row block runs that block's MFMAs only (the same loads
            // and barriers): a 6-row tile no longer costs a full one.
            uint32_t live_blocks = 0;  // bit i: block i has a row
#pragma unroll
            for (int i = 0; i < FM; ++i)
                live_blocks |= (__builtin_amdgcn_ballot_w64(srow[wm * WTM + i * BR + (lane % BR)] >= 0) != 0)
                                << i;
            if constexpr (FM >= 2) {
                if (live_blocks == 1u) run_tile(std::integral_constant<int, 1>{});
                else run_tile(fm_all);
            } else {
                run_tile(fm_all);
            }
            if constexpr (NW == 8) __builtin_amdgcn_s_setprio(0);
        }
    } else if (nt > 0) {
        // Fallback (the union does not fit the stage): the 256 source rows of
        // up to G taps at a time are staged at rows g * TM + r of the whole A
        // area (both buffers), with every global load of the round in flight
        // together; the round's steps then run from LDS, each step's weights
        // loaded while the previous step's MFMAs run.
        constexpr int UPT = (TM * kSegs + NT - 1) / NT;
        constexpr int GA = NBUF * STAGE / (TM * GEO::PITCH);
        // taps per round: <= 56 VGPRs of loads, and at most 8 (a longer round
        // is not unrolled, and its register arrays would go to memory)
        constexpr int G0 = GA < 14 / UPT ? GA : 14 / UPT;
        constexpr int G = G0 < 8 ? G0 : 8;
        static_assert(G >= 1 && G * TM * GEO::PITCH <= NBUF * STAGE, "fallback rounds fit the A area");
        for (int kc = 0; kc < kch; ++kc) {
            const int64_t koff = (int64_t)kc * KC * ES;
            uint32_t m = tile_mask;
            while (m) {
                int og[G];  // the round's taps (-1 past the last)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    og[g] = m ? __ffs(m) - 1 : -1;
                    m &= m - 1;  // no-op once m is 0
                }
                u32x4 v[G][UPT];
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int j = 0; j < UPT; ++j) {
                        const int u = j * NT + tid;
                        v[g][j] = zero4;
                        if (og[g] < 0 || (TM * kSegs % NT != 0 && u >= TM * kSegs)) continue;
                        const int32_t src = src_of(og[g], u >> 2);
                        if (src >= 0)
                            v[g][j] = *reinterpret_cast<const u32x4*>(xb + (int64_t)src * a.cin * ES +
                                                                      koff + (u & 3) * 16);
                    }
                Slot bs[2];
                load_b(og[0], kc, bs[0]);
                lds_barrier();  // every wave is done reading the A area
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int j = 0; j < UPT; ++j) {
                        const int u = j * NT + tid;
                        if (og[g] < 0 || (TM * kSegs % NT != 0 && u >= TM * kSegs)) continue;
                        Au[GEO::seg_pos(g * TM + (u >> 2), u & 3)] = v[g][j];
                    }
                lds_barrier();
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (og[g] < 0) break;
                    if (g + 1 < G && og[g + 1 < G ? g + 1 : g] >= 0)
                        load_b(og[g + 1 < G ? g + 1 : g], kc, bs[(g + 1) & 1]);
                    int sl[FM];
#pragma unroll
                    for (int i = 0; i < FM; ++i)
                        sl[i] = GEO::key(g * TM + wm * WTM + i * BR + (lane % BR));
                    AFrag af;
                    read_frags(0, sl, af, fm_all);
                    mma_step(af, bs[g & 1], fm_all);
                }
            }
        }
    }

    // ---- epilogue LayerNorm -> modulation -> SiLU over whole output rows
    // (TN == cout: the tile holds every channel of its rows).  The rounded
    // conv outputs go to an F32 LDS tile (in NPN passes over row halves when
    // the whole tile does not fit the A stage); groups of TN/4 lanes then
    // take one row each (four channels per lane, four rows in flight per
    // lane group), with group-local shuffles for the mean and the biased
    // variance.
    if constexpr (norm_epilogue_fits<GEO, TN>()) if (a.epi_mode == SPC_EPI_NORM_MOD_SILU) {
        constexpr int FP = TN + 4;           // f32 row pitch (16-byte multiple)
        constexpr int NPN = TM * FP * 4 <= ABYTES ? 1 : 2;  // passes
        constexpr int RPN = TM / NPN;        // tile rows per pass
        static_assert(RPN * FP * 4 <= ABYTES && RPN % 32 == 0, "f32 output tile fits the A stage");
        constexpr int G = TN / 4;            // lanes per row
        constexpr int RW = 64 / G;           // rows per wave at a time
        constexpr int RB = 4;                // row groups in flight per lane
        static_assert(RPN % (NW * RW * RB) == 0, "norm epilogue geometry");
        float* of = reinterpret_cast<float*>(Au);
        const int gl = lane % G;
        const int c0 = 4 * gl;
        char* yb = static_cast<char*>(a.y);
#pragma unroll
        for (int p = 0; p < NPN; ++p) {
        lds_barrier();  // every wave is done with the A stage / the previous pass
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rl = wm * WTM + i * BR + (lane % BR);
            if (wm * WTM + i * BR < p * RPN || wm * WTM + i * BR >= (p + 1) * RPN) continue;
#pragma unroll
            for (int c = 0; c < FC; ++c)
#pragma unroll
                for (int g = 0; g < M::NRUN; ++g) {
                    const int cl = wn * WTN + c * BC + M::run(lane, g);
                    *reinterpret_cast<floatx4*>(of + (rl - p * RPN) * FP + cl) =
                        floatx4{M::round(acc[i][c][4 * g]), M::round(acc[i][c][4 * g + 1]),
                                M::round(acc[i][c][4 * g + 2]), M::round(acc[i][c][4 * g + 3])};
                }
        }
        lds_barrier();
        for (int it = 0; it < RPN / (NW * RW * RB); ++it) {
            float v[RB][4];
            int32_t t[RB];
            float s[RB], q[RB];
#pragma unroll
            for (int k = 0; k < RB; ++k) {
                const int r = ((it * RB + k) * NW + wave) * RW + lane / G;
                t[k] = srow[p * RPN + r];
                const floatx4 f = *reinterpret_cast<const floatx4*>(of + r * FP + c0);
                v[k][0] = f.x; v[k][1] = f.y; v[k][2] = f.z; v[k][3] = f.w;
                s[k] = (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
            }
#pragma unroll
            for (int off = G / 2; off > 0; off >>= 1)
#pragma unroll
                for (int k = 0; k < RB; ++k) s[k] += __shfl_xor(s[k], off);
#pragma unroll
            for (int k = 0; k < RB; ++k) {
                const float mean = s[k] / (float)TN;
                q[k] = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[k][e] -= mean;
                    q[k] += v[k][e] * v[k][e];
                }
            }
#pragma unroll
            for (int off = G / 2; off > 0; off >>= 1)
#pragma unroll
                for (int k = 0; k < RB; ++k) q[k] += __shfl_xor(q[k], off);
#pragma unroll
            for (int k = 0; k < RB; ++k) {
                if (t[k] < 0) continue;
                const float rstd = 1.0f / sqrtf(q[k] / (float)TN + a.epi_eps);
                const int64_t b = min(max((int64_t)a.coords[(int64_t)t[k] * 4], (int64_t)0), a.n_batch - 1);
                const floatx4 sc = *reinterpret_cast<const floatx4*>(a.epi_scale + b * a.cout + c0);
                const floatx4 sh = *reinterpret_cast<const floatx4*>(a.epi_shift + b * a.cout + c0);
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float u = M::round(v[k][e] * rstd);           // norm2 (LayerNorm32)
                    const float m = M::round(M::round(u * M::round(1.0f + sc[e])) + sh[e]);
                    o[e] = silu_f32(m);                                  // SiLU
                }
                char* dst = yb + ((int64_t)t[k] * a.cout + c0) * ES;
                if constexpr (ES == 4) {
                    *reinterpret_cast<floatx4*>(dst) = floatx4{o[0], o[1], o[2], o[3]};
                } else {
                    *reinterpret_cast<u32x2*>(dst) =
                        u32x2{(uint32_t)M::cvt(o[0]) | ((uint32_t)M::cvt(o[1]) << 16),
                              (uint32_t)M::cvt(o[2]) | ((uint32_t)M::cvt(o[3]) << 16)};
                }
            }
        }
        }  // passes
        return;
    }

    // ---- per-wave epilogue (staged fast path, 16-bit output, no norm): the
    // wave's rounded block goes to its private LDS region (with two buffers
    // the last chunk reads only its own, so the other one is free) and back as
    // whole 16-byte pieces of its rows, which leave with coalesced
    // non-temporal stores -- no barrier, so early waves store while the
    // late ones finish their MFMAs.  Same values as the tile epilogue below.
    if constexpr (PWE) if (dma) {
        const int freebuf = ((kch - 1) & 1) ^ 1;  // (two buffers)
        char* reg = wave < PW_IN_STAGE
                        ? reinterpret_cast<char*>(Au + freebuf * STAGE) + wave * PW_BYTES
                        : pw_extra + (wave - PW_IN_STAGE) * PW_BYTES;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rl = i * BR + (lane % BR);
#pragma unroll
            for (int c = 0; c < FC; ++c)
#pragma unroll
                for (int g = 0; g < M::NRUN; ++g) {
                    const int cl = c * BC + M::run(lane, g);
                    *reinterpret_cast<u32x2*>(reg + rl * PW_PITCH + cl * ES) =
                        u32x2{(uint32_t)M::cvt(acc[i][c][4 * g]) | ((uint32_t)M::cvt(acc[i][c][4 * g + 1]) << 16),
                              (uint32_t)M::cvt(acc[i][c][4 * g + 2]) | ((uint32_t)M::cvt(acc[i][c][4 * g + 3]) << 16)};
                }
        }
        // the reads below take other lanes' writes: keep the compiler from
        // moving them up, and let the writes land
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        constexpr int UPW = WTN * ES / 16;     // 16-byte pieces per row of the block
        constexpr int NUW = WTM * UPW / 64;    // per lane
        static_assert(WTM * UPW % 64 == 0, "per-wave store geometry");
        char* yb = static_cast<char*>(a.y);
        const int64_t col = co0 + wn * WTN;
        int32_t tt[NUW];
        u32x4 vv[NUW];
#pragma unroll
        for (int k = 0; k < NUW; ++k) {
            const int c = k * 64 + lane;
            const int r = c / UPW;
            tt[k] = srow[wm * WTM + r];
            vv[k] = *reinterpret_cast<const u32x4*>(reg + r * PW_PITCH + (c % UPW) * 16);
        }
        if (a.epi_mode == SPC_EPI_RESIDUAL) {
            // y = dt(dt(conv + bias) + residual), as in the tile epilogue
#pragma unroll
            for (int k = 0; k < NUW; ++k) {
                int32_t rr = tt[k];
                if (a.residual_rows && rr >= 0) {
                    const int32_t v = a.residual_rows[rr];
                    rr = (v >= 0 && v < a.n_residual) ? v : -1;
                }
                const u32x4 rv = rr >= 0 ? *reinterpret_cast<const u32x4*>(
                                               static_cast<const char*>(a.residual) +
                                               ((int64_t)rr * a.cout + col) * ES + ((k * 64 + lane) % UPW) * 16)
                                         : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = M::unpack(vv[k][e], 0) + M::unpack(rv[e], 0);
                    const float hi = M::unpack(vv[k][e], 1) + M::unpack(rv[e], 1);
                    vv[k][e] = (uint32_t)M::cvt(lo) | ((uint32_t)M::cvt(hi) << 16);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < NUW; ++k)
            if (tt[k] >= 0)
                __builtin_nontemporal_store(
                    vv[k], reinterpret_cast<u32x4*>(yb + ((int64_t)tt[k] * a.cout + col) * ES +
                                                    ((k * 64 + lane) % UPW) * 16));
        return;
    }

    // ---- epilogue: + bias in F32, one rounding.  Each lane holds four runs
    // of four consecutive channels of one row; they go to an LDS output
    // tile (8-byte writes, 16 in f32), then whole rows leave with coalesced
    // 16-byte stores.
    constexpr int OPITCH = TN * ES + 8;  // bytes per output-tile row in LDS
    constexpr int NPASS = TM * OPITCH <= ABYTES ? 1 : TM / 2 * OPITCH <= ABYTES ? 2 : 4;  // wide f32 tiles go in parts
    constexpr int RPP = TM / NPASS;      // tile rows per pass
    static_assert(RPP * OPITCH <= ABYTES && RPP % 32 == 0, "output tile fits the A stage");
    constexpr int UPR = TN * ES / 16;    // 16-byte units per output row
    char* ob = reinterpret_cast<char*>(Au);
    char* yb = static_cast<char*>(a.y);
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
        lds_barrier();  // every wave is done with the A stage / the previous pass
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rl = wm * WTM + i * BR + (lane % BR);
            if (wm * WTM + i * BR < p * RPP || wm * WTM + i * BR >= (p + 1) * RPP) continue;
#pragma unroll
            for (int c = 0; c < FC; ++c) {
#pragma unroll
                for (int g = 0; g < M::NRUN; ++g) {
                    const int cl = wn * WTN + c * BC + M::run(lane, g);
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[i][c][4 * g + e];
                    char* dst = ob + (rl - p * RPP) * OPITCH + cl * ES;
                    if constexpr (ES == 4) {
                        *reinterpret_cast<float2*>(dst) = float2{v[0], v[1]};
                        *reinterpret_cast<float2*>(dst + 8) = float2{v[2], v[3]};
                    } else {
                        *reinterpret_cast<u32x2*>(dst) =
                            u32x2{(uint32_t)M::cvt(v[0]) | ((uint32_t)M::cvt(v[1]) << 16),
                                  (uint32_t)M::cvt(v[2]) | ((uint32_t)M::cvt(v[3]) << 16)};
                    }
                }
            }
        }
        lds_barrier();
        // all LDS reads first, then the stores
        constexpr int NU = RPP * UPR / NT;
        static_assert(RPP * UPR % NT == 0, "store geometry");
        int32_t tt[NU];
        u32x4 vv[NU];
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int c = tid + k * NT;
            const int r = c / UPR;
            const int q = c - r * UPR;
            tt[k] = srow[p * RPP + r];
            const char* src = ob + r * OPITCH + q * 16;
            const u32x2 lo = *reinterpret_cast<const u32x2*>(src);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 8);
            vv[k] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
        if (a.epi_mode == SPC_EPI_RESIDUAL) {
            // y = dt(dt(conv + bias) + residual): the rounded conv output
            // plus the residual row, added in F32 and rounded once more
            u32x4 rv[NU];
            int32_t rr[NU];
#pragma unroll
            for (int k = 0; k < NU; ++k) {
                rr[k] = tt[k];
                if (a.residual_rows && tt[k] >= 0) {
                    const int32_t v = a.residual_rows[tt[k]];
                    rr[k] = (v >= 0 && v < a.n_residual) ? v : -1;
                }
            }
#pragma unroll
            for (int k = 0; k < NU; ++k) {
                const int q = (tid + k * NT) % UPR;
                rv[k] = rr[k] >= 0 ? *reinterpret_cast<const u32x4*>(
                                         static_cast<const char*>(a.residual) +
                                         ((int64_t)rr[k] * a.cout + co0) * ES + q * 16)
                                   : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int k = 0; k < NU; ++k) {
                if constexpr (ES == 4) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        vv[k][e] = __float_as_uint(__uint_as_float(vv[k][e]) + __uint_as_float(rv[k][e]));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float lo = M::unpack(vv[k][e], 0) + M::unpack(rv[k][e], 0);
                        const float hi = M::unpack(vv[k][e], 1) + M::unpack(rv[k][e], 1);
                        vv[k][e] = (uint32_t)M::cvt(lo) | ((uint32_t)M::cvt(hi) << 16);
                    }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            const int c = tid + k * NT;
            const int q = c % UPR;
            if (tt[k] >= 0)
                __builtin_nontemporal_store(
                    vv[k], reinterpret_cast<u32x4*>(yb + ((int64_t)tt[k] * a.cout + co0) * ES + q * 16));
        }
    }
}

template <typename T, bool Q8, bool PACKED, int NTAPS, int TN, int WM, int WN, typename GEO = GeoWide>
hipError_t launch_conv(hipStream_t s, ConvArgs a) {
    constexpr int TM = GEO::TM;
    const int64_t tiles_m = ceil_div(a.n_out, TM);
    a.tiles_n = a.cout / TN;
    a.total_tiles = tiles_m * a.tiles_n;
    a.heavy_tiles = (a.n_out % TM ? tiles_m - 1 : tiles_m) * a.tiles_n;
    a.tiles_per_xcd = ceil_div(a.heavy_tiles, 8);
    const int64_t wbytes = (int64_t)NTAPS * max(1, a.n_classes) * a.cin * a.cout * (Q8 ? 1 : (int)sizeof(T));
    a.col_major = a.tiles_n > 1 && wbytes > (2 << 20);
    const int64_t grid = a.tiles_per_xcd * 8 + (a.total_tiles - a.heavy_tiles);
    if (grid == 0) return hipSuccess;
    if (a.epi_mode == SPC_EPI_NORM_MOD_SILU && !norm_epilogue_fits<GEO, TN>())
        return hipErrorInvalidValue;  // the tile cannot hold the epilogue's rows
    // the plan buffer holds the wide plans, then the small ones
    if (a.plan && !GEO::WIDE_PLAN)
        a.plan = static_cast<const char*>(a.plan) + plan_wide_bytes(a.n_out, NTAPS);
    conv_kernel<T, Q8, PACKED, NTAPS, TN, WM, WN, 4, GEO><<<(unsigned)grid, WM * WN * 64, 0, s>>>(a);
    return hipGetLastError();
}

// The stride-2 conv's 64-row tiles over four buffers (GeoQuad), picked by
// shape: up to four 64-byte channel chunks (C_in <= 128 in 16-bit, 64 in
// f32) and every tile on its own CU in one round (4 ellipsoid shells' 11,774 coarse
// rows at C_out 128: 184 tiles).  Same wave layouts as the small tiles.
template <typename T, bool Q8, bool PACKED, int NTAPS>
bool use_quad_tiles(const ConvArgs& a, int tn) {
    if constexpr (NTAPS != 8) {
        return false;
    } else {
        const int64_t kch = (int64_t)a.cin * (int64_t)sizeof(T) / 64;
        // by shape, also under a forced geometry that does not apply here
        return a.geometry != SPC_TILES_WIDE && a.geometry != SPC_TILES_SMALL &&
               a.epi_mode != SPC_EPI_NORM_MOD_SILU && kch <= 4 &&
               ceil_div(a.n_out, GeoQuad::TM) * (a.cout / tn) <= a.num_cu;
    }
}

// Small tiles (GeoSmall: 128 rows, 64 for stride-2; three 4-wave
// workgroups per CU, two at TN = 128): TN = largest of {128, 64, 32} dividing cout, halved
// while the narrower tiles still fit on the device in one round; waves 2 x 2
// (64 x 64 / 64 x 32 wave tiles; 32 x 64 / 32 x 32 for 64-row tiles), 4 x 1
// (32 x 32) at TN = 32, 2 x 1 for 64-row tiles; 1 x 4 (128 x 32) for Q8_0
// at TN = 128.
template <typename T, bool Q8, bool PACKED, int NTAPS>
hipError_t dispatch_small(hipStream_t s, const ConvArgs& a) {
    using G = GeoSmall<NTAPS>;
    const int64_t tiles_m = ceil_div(a.n_out, G::TM);
    int tn = a.cout % 128 == 0 ? 128 : a.cout % 64 == 0 ? 64 : 32;
    while (tn > 32 && tiles_m * (a.cout / (tn / 2)) <= a.num_cu) tn /= 2;
    if (a.epi_mode == SPC_EPI_NORM_MOD_SILU) tn = a.cout;  // 32 or 64 here (one tile per row)
    if constexpr (NTAPS == 8) {
        if (use_quad_tiles<T, Q8, PACKED, NTAPS>(a, tn)) {
            if (tn == 128) return launch_conv<T, Q8, PACKED, NTAPS, 128, 2, 4, GeoQuad>(s, a);
            if (tn == 64) return launch_conv<T, Q8, PACKED, NTAPS, 64, 2, 2, GeoQuad>(s, a);
            return launch_conv<T, Q8, PACKED, NTAPS, 32, 2, 1, GeoQuad>(s, a);
        }
    }
    if (tn == 128) {
        // Q8_0: 4 waves of 128 x 32, so each in-register dequantised B
        // fragment feeds four MFMAs and no two waves dequantise the same one
        if constexpr (Q8 && G::TM == 128) return launch_conv<T, Q8, PACKED, NTAPS, 128, 1, 4, G>(s, a);
        else return launch_conv<T, Q8, PACKED, NTAPS, 128, 2, 2, G>(s, a);
    }
    if (tn == 64) return launch_conv<T, Q8, PACKED, NTAPS, 64, 2, 2, G>(s, a);
    if constexpr (G::TM == 128) return launch_conv<T, Q8, PACKED, NTAPS, 32, 4, 1, G>(s, a);
    else return launch_conv<T, Q8, PACKED, NTAPS, 32, 2, 1, G>(s, a);
}


// Which geometry a conv runs.  a.geometry forces one (1 wide, 2 small);
// otherwise the small tiles take the shapes where their single stage buffer
// costs nothing because co-resident workgroups hide each other's staging:
//   - the 8-tap stride-2 conv (256 coarse rows reference ~1,360 fine rows,
//     beyond the wide stage: 29.8 -> 11.6 us for 128 -> 128 over 62,710
//     fine rows);
//   - one or two channel chunks per tile (C_in <= 64 in 16-bit, <= 32 in
//     f32) into at most 64 output channels, where a wide tile is mostly
//     setup and staging latency (the mesh levels: 31.8 -> 23.3 us at 128^3
//     C=64, 50.8 -> 38.7 us at 256^3 C=32);
//   - 128-column tiles that need more than one round of the CUs, so the
//     workgroups sharing a CU drift apart (SubM 1024 -> 1024 over 11,774
//     rows: 627 -> 572 us; 128 -> 1024: 105 -> 89 us).
// A single round of long wide tiles stays wide: the double-buffered stage
// overlaps every chunk's staging with the MFMAs, which the small tiles'
// synchronised workgroups cannot (C=128 over 62,710 rows: 57 vs 104 us;
// f32 C=64 over 21,766 rows: 62.9 vs 65.2 us).
// Packed weights, 27 or 8 taps (the dense 1 x 1 x 1 conv keeps the wide
// tiles, as do weight classes, the 96- / 192-column tiles and the norm
// epilogue over 128 channels).
template <typename T, bool Q8, bool PACKED, int NTAPS>
bool use_small_tiles(const ConvArgs& a) {
    if constexpr (!PACKED || NTAPS == 1) {
        return false;
    } else {
        if (a.epi_mode == SPC_EPI_NORM_MOD_SILU && a.cout > 64) return false;
        if (a.geometry == SPC_TILES_WIDE || a.geometry == SPC_TILES_SMALL) return a.geometry == SPC_TILES_SMALL;
        if (a.class_rows > 0) return false;
        if (NTAPS == 8) return true;
        const int64_t kch = (int64_t)a.cin * (int64_t)sizeof(T) / 64;
        // short rows into narrow outputs only: with 128 output columns the
        // wide tiles' double-buffered stage wins (C_in 64 -> C_out 128 over
        // 62,710 rows: 53.7 us small, 29.8 us wide; C_in 32: 29.4 / 19.6 us)
        if (kch <= 2) return a.cout <= 64;
        const int64_t tiles_m = ceil_div(a.n_out, GeoWide::TM);
        return a.cout % 128 == 0 && tiles_m * (a.cout / 128) > a.num_cu;
    }
}

// Tall tiles (GeoTall: 256 rows over one 559-row stage, three 4-wave
// workgroups per CU): the SubM convs whose rows are one 64-byte chunk
// (C_in = 32 in 16-bit, 16 in f32) and whose C_out is 32 or 64 -- where a
// 128-row small tile is mostly setup and staging latency and only three of
// them fit a CU.  Forced (SPC_TILES_TALL), any packed 27-tap conv with
// 32-column multiples except the norm epilogue and weight classes.  Waves
// 4 x 1 of 64 x 32 (64 x 64 wave tiles would spill at the 168-register
// budget of three workgroups per CU; C_out = 64 runs two column tiles).
template <typename T, bool Q8, bool PACKED, int NTAPS>
bool use_tall_tiles(const ConvArgs& a) {
    if constexpr (!PACKED || NTAPS != 27) {
        return false;
    } else {
        if (a.epi_mode == SPC_EPI_NORM_MOD_SILU || a.class_rows > 0 || a.cout % 32 != 0) return false;
        if (a.geometry != SPC_TILES_AUTO) return a.geometry == SPC_TILES_TALL;
        return (int64_t)a.cin * (int64_t)sizeof(T) == 64 && a.cout <= 64;
    }
}

template <typename T, bool Q8, bool PACKED, int NTAPS>
hipError_t dispatch_tall(hipStream_t s, const ConvArgs& a) {
    return launch_conv<T, Q8, PACKED, NTAPS, 32, 4, 1, GeoTall>(s, a);
}

// Wide tiles: TN = largest of {128, 64, 32} dividing cout, halved while the
// narrower tiles still fit on the device in one round (small row counts
// would leave compute units idle); 8 waves as 4x2 (64x64 wave tiles), 4x2
// (64x32) or 8x1 (32x32).  Q8_0 weights use 4 waves of 128x64: each
// in-register dequantised B fragment then feeds four MFMAs instead of two.
template <typename T, bool Q8, bool PACKED, int NTAPS>
hipError_t dispatch_tn(hipStream_t s, const ConvArgs& a) {
    if (a.epi_mode == SPC_EPI_NORM_MOD_SILU && a.cout != 32 && a.cout != 64 && a.cout != 128)
        return hipErrorInvalidValue;  // the epilogue's lane groups need one 32/64/128-column tile
    if constexpr (PACKED && NTAPS != 1) {
        if constexpr (NTAPS == 27)
            if (use_tall_tiles<T, Q8, PACKED, NTAPS>(a)) return dispatch_tall<T, Q8, PACKED, NTAPS>(s, a);
        if (use_small_tiles<T, Q8, PACKED, NTAPS>(a)) return dispatch_small<T, Q8, PACKED, NTAPS>(s, a);
    }
    const int64_t tiles_m = ceil_div(a.n_out, GeoWide::TM);
    int tn = a.cout % 128 == 0 ? 128 : a.cout % 64 == 0 ? 64 : 32;
    while (tn > 32 && tiles_m * (a.cout / (tn / 2)) <= a.num_cu) tn /= 2;
    // a ragged last round of 128-column tiles (e.g. 368 tiles on 256 compute
    // units: two rounds, the second 44% full) costs a whole round; 64-column
    // tiles (about 0.6 of the time each) pay off when they need fewer than
    // 10/6 as many rounds (SubM 1024 -> 1024 over 11774 rows: 627 -> 591 us)
    if constexpr (!Q8) {
        if (tn == 128) {
            const int64_t r128 = ceil_div(tiles_m * (a.cout / 128), a.num_cu);
            const int64_t r64 = ceil_div(tiles_m * (a.cout / 64), a.num_cu);
            if (r64 * 6 < r128 * 10) tn = 64;
        }
    }
    if (a.epi_mode == SPC_EPI_NORM_MOD_SILU) tn = a.cout;  // one tile covers the row
    // widths 128 does not divide but 192 does (the mesh decoder's 768 / 4):
    // one 192-column tile of 4 waves (2 x 2, 128x96 wave tiles, one per
    // SIMD) instead of three 64-column tiles of 64x32 wave tiles, which read
    // each A fragment for half the MFMA work and are LDS-bound.  Packed
    // 16-bit weights, and only once the row tiles alone fill the device.
    if constexpr (!Q8 && PACKED && sizeof(T) == 2) {
        if (a.cout % 192 == 0 && a.cout % 128 != 0 && a.epi_mode != SPC_EPI_NORM_MOD_SILU &&
            tiles_m * (a.cout / 192) >= a.num_cu)
            return launch_conv<T, Q8, PACKED, NTAPS, 192, 2, 2>(s, a);
        // 96 (the mesh decoder's 768 / 8): eight waves of 64x48 (two per
        // SIMD, weights loaded per 16-channel block) instead of three
        // 32-column tiles of 32x32 wave tiles
        if (a.cout % 96 == 0 && a.cout % 64 != 0 && a.epi_mode != SPC_EPI_NORM_MOD_SILU &&
            tiles_m * (a.cout / 96) >= a.num_cu)
            return launch_conv<T, Q8, PACKED, NTAPS, 96, 4, 2>(s, a);
    }
    if (tn == 128) {
        if constexpr (Q8) return launch_conv<T, Q8, PACKED, NTAPS, 128, 2, 2>(s, a);
        else return launch_conv<T, Q8, PACKED, NTAPS, 128, 4, 2>(s, a);
    }
    if (tn == 64) return launch_conv<T, Q8, PACKED, NTAPS, 64, 4, 2>(s, a);
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
