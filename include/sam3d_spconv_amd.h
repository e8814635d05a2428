/*
 * sam3d_spconv_amd.h -- C ABI of the MI355X (gfx950) sparse-voxel
 * convolution library (libsam3d_spconv_amd.so).
 *
 * Scope: the submanifold 3x3x3 and stride-2 SparseConv3d path of SAM 3D
 * Objects -- kernel-map build, gather -> implicit GEMM -> store, stride-2
 * downsample / subdivide maps, Q8_0 weights, scatter-mean.  Citations are
 * relative to the reference repository (Asher-1/sam-3d-objects-ggml):
 *   PATCH = cpp_ggml/third_party/ggml-patches/0001-sam3d-ggml-combined.patch
 *   SRC   = cpp_ggml/src
 *   SP    = sam3d_objects/model/backbone/tdfy_dit/modules/sparse
 *
 * Conventions
 *   - Every buffer is caller-owned device memory (hipMalloc / torch).  The
 *     library allocates nothing at run time; scratch space comes from a
 *     caller-owned workspace whose size the *_workspace_bytes queries
 *     return.  The exceptions, one per device for the life of the process:
 *     the spconv bridge's packed weights, padded rows and tile-plan cache
 *     (sam3d_spconv_f16_forward, whose signature has no workspace: grown
 *     with hipMalloc by the calls that need them) and the 56 MiB static map
 *     scratch of spc_map_build_noalloc (reserved on every device the library
 *     runs on) -- documented at their entry points.
 *   - Calls are asynchronous on `stream` (a hipStream_t; 0 = null stream)
 *     unless documented as synchronising.  Calls on one stream are ordered;
 *     separate workspaces make calls on different streams independent.
 *   - Every entry point returns an spc_status; spc_last_error() describes
 *     the most recent failure of the calling thread.
 *   - Coordinates are int32 (b, x, y, z) rows.  The GPU key packing accepts
 *     b in [0, 262144) and x, y, z in [0, 32768); anything else is
 *     SPC_BAD_COORD (SparseTensor's contract is [0, 1023], SP/basic.py:33).
 *   - Offsets o = kd*9 + kh*3 + kw with (dx,dy,dz) = (o/9-1, (o/3)%3-1,
 *     o%3-1); centre tap o = 13 (SRC/sparse_ops.cpp:108).
 */
#ifndef SAM3D_SPCONV_AMD_H
#define SAM3D_SPCONV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* spc_stream_t; /* hipStream_t */

typedef enum {
    SPC_OK = 0,
    SPC_BAD_SHAPE = 1,   /* sizes / channel counts the kernels do not support   */
    SPC_BAD_COORD = 2,   /* coordinate outside the accepted range               */
    SPC_DUP_COORD = 3,   /* duplicate coordinate where uniqueness is required   */
    SPC_OOM = 4,         /* workspace too small                                 */
    SPC_HIP_ERROR = 5,   /* a HIP runtime call failed                           */
    SPC_BAD_ARG = 6      /* null pointer / unknown enum value                   */
} spc_status;

typedef enum { SPC_F32 = 0, SPC_F16 = 1, SPC_BF16 = 2, SPC_Q8_0 = 3 } spc_dtype;

/* Map-build flags. */
#define SPC_MAP_MESH 1u /* build_mesh_conv_table semantics: coords must lie in
                           [0, resolution) and be unique (SRC/sparse_ops.cpp:312-329) */
#define SPC_MAP_SYNC 2u /* synchronise `stream` and return the device-side status */

/* Index-table layouts accepted by spc_sparse_conv. */
#define SPC_IDX_TOKEN_MAJOR 0  /* [n_out, ntaps]; SRC/sparse_ops.cpp:102-116   */
#define SPC_IDX_OFFSET_MAJOR 1 /* [ntaps, n_out]; SRC/sparse_ops.cpp:124-133   */

/* Weight layouts.  spc_sparse_conv takes SPC_W_KRSC or SPC_W_PACKED;
 * spc_conv_pack_weights reads SPC_W_KRSC, SPC_W_TCK or SPC_W_TKC. */
#define SPC_W_KRSC 0   /* [cout, ntaps, cin]: spconv KRSC = ggml op row format
                          (PATCH:241-243; cpp_ggml/scripts/gguf_schema.py:330-338) */
#define SPC_W_PACKED 1 /* MFMA fragment order, made by spc_conv_pack_weights        */
#define SPC_W_TCK 2    /* [ntaps, cout, cin]: mesh-decoder GGUF rows, one (Cout,Cin)
                          matrix per offset (cpp_ggml/scripts/convert_sam3d_to_gguf.py:
                          508-511; SRC/mesh_decoder_graph.cpp:285-289,334-337)      */
#define SPC_W_TKC 3    /* [ntaps, cin, cout]: w[o][ci][co].  With ntaps = 1 this is the
                          1x1x1 skip conv's raw view of its saved [cout,1,1,1,cin]
                          buffer as (cin, cout) (SRC/mesh_decoder_graph.cpp:349-376) */

const char* spc_last_error(void);
const char* spc_status_string(int status);
int spc_version(void);

/* ------------------------------------------------------------------------
 * Kernel map (submanifold 3x3x3 neighbour tables).
 * Replaces SlatTables::build's conv tables (SRC/sparse_ops.cpp:93-155;
 * declared SRC/sparse_ops.hpp:24-39,46-47) and build_mesh_conv_table
 * (SRC/sparse_ops.cpp:312-346).  Bit-exact outputs:
 *   token_major  [n*27]  row of coord+delta(o) in the same batch, else n
 *   offset_major [27*n]  the same, offset-major, -1 when missing
 *   mask_sorted  [n]     27-bit valid-tap masks in stable ascending order
 *   argsort      [n]     std::stable_sort permutation of tokens by mask
 *   mask_natural [n]     the masks in token order (not a reference table)
 * Any output pointer may be NULL.  Duplicate coords without SPC_MAP_MESH
 * follow std::map::emplace: the first row owns the key, later duplicates
 * keep 27 sentinels and mask 0.  `resolution` is only read with
 * SPC_MAP_MESH.  Device-side errors (BAD_COORD, DUP_COORD) are returned
 * only with SPC_MAP_SYNC; otherwise read them with spc_read_status.
 * ------------------------------------------------------------------------ */
size_t spc_map_workspace_bytes(int64_t n);
int spc_map_build(spc_stream_t stream, const int32_t* coords, int64_t n, int32_t resolution,
                  uint32_t flags, int32_t* token_major, int32_t* offset_major,
                  int32_t* mask_sorted, int32_t* argsort, int32_t* mask_natural,
                  void* workspace, size_t workspace_bytes);

/* spc_map_build without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No reference counterpart.  The
 * scratch is a library-owned static device array of 56 MiB per device,
 * held until the process ends; n must be at most 1,048,576 (2^20) voxels,
 * larger n is SPC_BAD_SHAPE.  Same outputs, flags and semantics as
 * spc_map_build; device-side errors (BAD_COORD / DUP_COORD) are returned
 * with SPC_MAP_SYNC only (the status word lives in the shared scratch and
 * the next call rewrites it).  All calls on one device share the scratch:
 * calls that overlap on one device (other streams, other threads) race.
 * Calls no hipMalloc / hipFree. */
int spc_map_build_noalloc(spc_stream_t stream, const int32_t* coords, int64_t n,
                          int32_t resolution, uint32_t flags, int32_t* token_major,
                          int32_t* offset_major, int32_t* mask_sorted, int32_t* argsort,
                          int32_t* mask_natural);

/* spc_map_build over a dense grid [n_batch][R][R][R] of row ids (R =
 * resolution) instead of the hash table, for callers that bound the
 * coordinates: 0 <= b < n_batch and 0 <= x, y, z < R (others are BAD_COORD).
 * Same outputs, flags and duplicate rule (the first row owns a cell); each
 * lookup is one load.  The workspace holds the grid (4 bytes a cell, at
 * most 2^32 cells; the size query returns 0 and the build BAD_SHAPE beyond
 * that or for n_batch / resolution out of range).  No reference counterpart
 * (the reference's tables come from a std::map). */
size_t spc_map_dense_workspace_bytes(int64_t n, int64_t n_batch, int32_t resolution);
int spc_map_build_dense(spc_stream_t stream, const int32_t* coords, int64_t n, int64_t n_batch,
                        int32_t resolution, uint32_t flags, int32_t* token_major,
                        int32_t* offset_major, int32_t* mask_sorted, int32_t* argsort,
                        int32_t* mask_natural, void* workspace, size_t workspace_bytes);

/* Reads (and clears) the device status word of a map / downsample /
 * subdivide workspace.  Synchronises `stream`. */
int spc_read_status(spc_stream_t stream, void* workspace);

/* ------------------------------------------------------------------------
 * Stride-2 downsample map.  Replaces the coarse section of
 * SlatTables::build (SRC/sparse_ops.cpp:27-81; fields SRC/sparse_ops.hpp:
 * 15-23) and SparseDownsample's unique/inverse (SP/spatial.py:20-65).
 * Coarse key (b, x/2, y/2, z/2); coarse rows in lexicographic key order.
 *   fine_to_coarse [nf]          coarse row of each fine row
 *   coarse_coords  [nc, 4]       int32 (b, x/2, y/2, z/2)
 *   children       [8*nc]        fine rows, ascending, compacted, padded nf
 *   counts         [nc] float    |children| + 1 (mean over the zero row too)
 *   stride2_taps   [nc*8]        fine row at tap k = (x&1)*4+(y&1)*2+(z&1),
 *                                nf if absent (input of the 2x2x2 stride-2
 *                                conv; duplicates at one tap -> DUP_COORD)
 * Output buffers are sized for the upper bound nc = nf; the call
 * synchronises `stream` and writes nc to *nc_out (host).  Fine coords must
 * satisfy 0 <= b < n_batch and 0 <= x,y,z < resolution (<= 32768).
 * ------------------------------------------------------------------------ */
size_t spc_downsample_workspace_bytes(int64_t nf);
int spc_downsample_map(spc_stream_t stream, const int32_t* coords, int64_t nf, int64_t n_batch,
                       int32_t resolution, int32_t* fine_to_coarse, int32_t* coarse_coords,
                       int32_t* children, float* counts, int32_t* stride2_taps,
                       int64_t* nc_out, void* workspace, size_t workspace_bytes);

/* Map of the transposed 2x2x2 stride-2 conv (SparseInverseConv3d after a
 * stride-2 SparseConv3d, SP/conv/conv_spconv.py:92-139): taps [nf*8] with
 * taps[f*8 + k(f)] = fine_to_coarse[f] for the fine row's own tap k(f) =
 * (x&1)*4 + (y&1)*2 + (z&1), every other entry nc.  Used as the token-major
 * index table of spc_sparse_conv with ntaps 8, n_out nf, n_in nc. */
int spc_stride2_inverse_taps(spc_stream_t stream, const int32_t* coords,
                             const int32_t* fine_to_coarse, int64_t nf, int64_t nc,
                             int32_t* taps);

/* Token-major table [8 n_parent * 27] of a tensor subdivided without
 * `keep` (child c = 8p + d, spc_subdivide_map), derived from the parents'
 * token-major table [n_parent * 27] (spc_map_build, not SPC_MAP_MESH):
 * the child at 2x + d + delta(o) is child e of the parent at x + j, per
 * axis j = floor((d + delta) / 2), e = d + delta - 2j, and exists exactly
 * when that parent does.  Bit-exact with spc_map_build's token_major on the
 * child coordinates (sentinel 8 n_parent), without the hash build.  No
 * reference counterpart: the reference rebuilds the table from the
 * subdivided coordinates (SRC/sparse_ops.cpp:312-371). */
int spc_subdivide_neighbors(spc_stream_t stream, const int32_t* parent_token_major,
                            int64_t n_parent, int32_t* child_token_major);

/* Merged-tap form of the 3x3x3 submanifold conv over a tensor subdivided
 * without `keep`, whose child features are copies of the parent rows
 * (SparseSubdivide, SP/spatial.py:120-127): child c = 8p + d (d = dx*4 +
 * dy*2 + dz) has a neighbour at offset k exactly when the parent at
 * floor((d + k) / 2) exists, so its 27 taps read only 8 parent rows, at
 * offsets j with j_a in {d_a - 1, d_a}.  y[c] = b + sum_t W'(d, t) h[q_t]
 * with W'(d, t) the sum of the W_k that land on parent offset t.  Writes
 * idx [64 n_parent] (idx[c*8 + t], t = ix*4 + iy*2 + iz at j_a = d_a - 1 +
 * i_a; -1 when missing) and the class-major row order row_perm
 * [8 class_rows] (perm[d*class_rows + i] = 8i + d, -1 for i >= n_parent),
 * class_rows a multiple of 256 and >= n_parent.  With spc_sparse_conv_
 * classes (ntaps 8, n_classes 8, n_in n_parent, n_out 8 class_rows) this
 * runs the child conv on the parent features with 8 instead of 27 taps.
 * No reference counterpart. */
int spc_subdivide_tap_classes(spc_stream_t stream, const int32_t* parent_token_major,
                              int64_t n_parent, int64_t class_rows, int32_t* idx,
                              int32_t* row_perm);

/* Index composition: out[i] = rows[idx[i]] for idx[i] in [0, n_rows), else
 * -1 (idx and out 16-byte aligned).  With idx a neighbour table over
 * subdivided children and rows the children's parent rows (the `parent`
 * output of spc_subdivide_map), a conv on the composed table reads the
 * parents' features directly: SparseSubdivide's child features are copies
 * of the parent rows (SP/spatial.py:120-127), so the result equals the conv
 * over the copied rows exactly, without writing the copies.  No reference
 * counterpart: the reference materialises the copies. */
int spc_compose_rows(spc_stream_t stream, const int32_t* idx, int64_t n, const int32_t* rows,
                     int64_t n_rows, int32_t* out);

/* ------------------------------------------------------------------------
 * Subdivide map.  Replaces subdivide_mesh_level (SRC/sparse_ops.cpp:
 * 348-371) and SparseSubdivide's coordinates (SP/spatial.py:108-124).
 * Child c = dx*4 + dy*2 + dz of parent p has coords (b, 2x+dx, 2y+dy, 2z+dz)
 * and row p*8+c; with `keep` ([8n] bytes, nonzero = keep) survivors stay in
 * parent-major order.  parent[m] = the parent row of each output row.
 * Outputs sized for 8n rows; writes the row count m to *m_out.  With
 * `keep` the call synchronises `stream` (m is read back) and returns the
 * device-side status (BAD_COORD: a parent coordinate outside [0, 2^14) or
 * a batch index out of range); without `keep`, m = 8n and the call
 * synchronises and returns that status only with SPC_MAP_SYNC -- otherwise
 * it returns once the kernels are queued and the status is read with
 * spc_read_status on the same workspace (the reference's subdivide,
 * SP/spatial.py:120-124, checks no range at all).
 * ------------------------------------------------------------------------ */
size_t spc_subdivide_workspace_bytes(int64_t n);
int spc_subdivide_map(spc_stream_t stream, const int32_t* coords, int64_t n, const uint8_t* keep,
                      uint32_t flags, int32_t* out_coords, int32_t* parent, int64_t* m_out,
                      void* workspace, size_t workspace_bytes);

/* ------------------------------------------------------------------------
 * Sparse convolution: gather -> implicit GEMM (MFMA) -> store.
 * Same arithmetic as the ggml CPU op ggml_compute_forward_sam3d_sparse_
 * conv_f16 (PATCH:217-265) -- F32 accumulation of bias + sum over valid
 * taps and channels, one rounding to the output dtype -- and the same
 * contract as the CUDA bridge sam3d_spconv_f16_forward (SPCONV bridge,
 * cpp_ggml/third_party/sam3d-spconv/include/sam3d_spconv_bridge.cuh:10-21),
 * for 27 taps (submanifold 3x3x3) and 8 taps (2x2x2 stride 2):
 *   y[t, co] = bias[co] + sum_{o, s = idx(t,o) in [0,n_in)} sum_c
 *              w[co, o, c] * x[s, c]
 *   dtype    SPC_F32 / SPC_F16 / SPC_BF16: x, y, bias (and w unless Q8_0)
 *   w_dtype  == dtype, or SPC_Q8_0 with dtype SPC_BF16
 *   w_layout SPC_W_KRSC: w is [cout, ntaps, cin] (Q8_0: int8 quants with
 *            w_scale = fp16 block scales [cout, ntaps, cin/32], as
 *            spc_q8_0_repack makes them from ggml blocks);
 *            SPC_W_PACKED: w from spc_conv_pack_weights (w_scale unused) --
 *            the fast path, each MFMA operand one contiguous load
 *   idx      SPC_IDX_TOKEN_MAJOR [n_out, ntaps] or SPC_IDX_OFFSET_MAJOR
 *            [ntaps, n_out]; entries outside [0, n_in) are skipped
 *   row_perm optional [n_out]: processing order; processing row r computes
 *            and writes output row row_perm[r].  Rows in lexicographic
 *            (natural) order are fastest: the kernel deduplicates the
 *            gathered rows of each 256-row tile.
 *   bias     may be NULL
 * Requires ntaps 27, 8 or 1, cin % 32 == 0, cout % 32 == 0, ntaps*cin*cout*4 < 2^31.  With ntaps 1
 * and idx NULL the map is the identity (n_in == n_out): the dense 1x1x1
 * conv y = x W^T + b of sparse_conv_1x1 (SRC/mesh_decoder_graph.cpp:349-384).
 * ------------------------------------------------------------------------ */
int spc_sparse_conv(spc_stream_t stream, int dtype, const void* x, int w_dtype, int w_layout,
                    const void* w, const void* w_scale, const void* bias, void* y,
                    const int32_t* idx, int idx_layout, const int32_t* row_perm, int64_t ntaps,
                    int64_t n_out, int64_t n_in, int64_t cin, int64_t cout);

/* Tile plan: the per-tile setup of the conv kernel (active tap set,
 * deduplicated source rows, slot table) for both tile geometries (the
 * 256-row tiles, then the small ones; see spc_conv_set_tile_geometry),
 * built once per index table and reused by every conv over it -- like the
 * map, it depends only on
 * (idx, idx_layout, row_perm, ntaps, n_out, n_in), not on channels or
 * weights.  spc_sparse_conv_plan takes the same arguments as
 * spc_sparse_conv plus a plan built from those same arguments (256-byte
 * aligned); a plan from other arguments gives wrong results.  No
 * reference counterpart: a cache of this library's kernel setup, in the
 * role of spconv's indice_key pair cache (SP/conv/conv_spconv.py:30-50). */
size_t spc_conv_plan_bytes(int64_t n_out, int64_t ntaps);
int spc_conv_plan(spc_stream_t stream, const int32_t* idx, int idx_layout,
                  const int32_t* row_perm, int64_t ntaps, int64_t n_out, int64_t n_in, void* plan,
                  size_t plan_bytes);
/* spc_conv_plan building only the given sections (SPC_PLAN_WIDE and / or
 * SPC_PLAN_SMALL) of a plan of the same size: a conv whose tile geometry
 * finds its section unbuilt sets its tiles up itself (same results,
 * slower), so callers that rebuild plans often (per call) build only the
 * geometry their convs run. */
#define SPC_PLAN_WIDE 1u
#define SPC_PLAN_SMALL 2u
int spc_conv_plan_sections(spc_stream_t stream, const int32_t* idx, int idx_layout,
                           const int32_t* row_perm, int64_t ntaps, int64_t n_out, int64_t n_in,
                           uint32_t sections, void* plan, size_t plan_bytes);
int spc_sparse_conv_plan(spc_stream_t stream, int dtype, const void* x, int w_dtype,
                         int w_layout, const void* w, const void* w_scale, const void* bias,
                         void* y, const int32_t* idx, int idx_layout, const int32_t* row_perm,
                         const void* plan, int64_t ntaps, int64_t n_out, int64_t n_in,
                         int64_t cin, int64_t cout);

/* Tile geometry of the conv kernel.  Every conv runs on one of three:
 *   SPC_TILES_WIDE   256-row tiles over an 895-row double-buffered stage,
 *                    one 8-wave workgroup per CU (long tiles: wide channels);
 *   SPC_TILES_SMALL  128-row tiles (64 for 8 taps) over a 511-row stage,
 *                    two or three 4-wave workgroups per CU (short tiles: small
 *                    channel counts, few rows, the stride-2 conv; a stride-2
 *                    conv of up to four 64-byte channel chunks whose tiles
 *                    fit the CUs in one round stages all its chunks at once
 *                    in four buffers, one 8-wave workgroup per CU);
 *   SPC_TILES_TALL   256-row tiles over a 559-row stage, three 4-wave
 *                    workgroups per CU (one-chunk rows: 16-bit C_in = 32 with
 *                    C_out 32 or 64); reads the wide tiles' plan section.
 * All give the same results.  By default (SPC_TILES_AUTO) each conv picks
 * by shape; spc_conv_set_tile_geometry forces one for every later conv of
 * the process (measurements, tests; initially from the environment
 * variable SPC_CONV_GEOMETRY = "wide" / "small" / "tall").  The small tiles
 * apply to packed weights with 27 or 8 taps, the tall ones to packed
 * weights with 27 taps and C_out a multiple of 32, without the norm
 * epilogue or weight classes (elsewhere a forced geometry that does not
 * apply leaves the choice by shape).  Plans (spc_conv_plan) hold the wide
 * and the small sections.  No reference counterpart. */
#define SPC_TILES_AUTO 0
#define SPC_TILES_WIDE 1
#define SPC_TILES_SMALL 2
#define SPC_TILES_TALL 3
int spc_conv_set_tile_geometry(int geometry);
/* The geometry (SPC_TILES_WIDE / SMALL / TALL) a conv with packed weights
 * and these arguments runs now (epi_mode a spc_epilogue_mode, class_rows 0
 * without weight classes); SPC_TILES_SMALL reads the small plan section,
 * the others the wide one. */
int spc_conv_tile_geometry(int dtype, int w_dtype, int64_t ntaps, int64_t n_out, int64_t cin,
                           int64_t cout, int64_t class_rows, int epi_mode);

/* Bytes of the SPC_W_PACKED form of ntaps x cout x cin weights of w_dtype
 * (Q8_0: quants then f32 scales), and the packer.  w_layout (SPC_W_KRSC,
 * SPC_W_TCK or SPC_W_TKC) says how w is stored.  Q8_0 quants (int8) come
 * with fp16 block scales w_scale, one per 32 consecutive stored channels,
 * which must run along cin: SPC_W_KRSC or SPC_W_TCK (SPC_W_TKC Q8_0 weights
 * are dequantised first, as the reference does, SRC/mesh_decoder_graph.cpp:
 * 370-372).  No reference counterpart: the packed form is this library's
 * operand layout. */
size_t spc_conv_packed_bytes(int w_dtype, int64_t ntaps, int64_t cin, int64_t cout);
int spc_conv_pack_weights(spc_stream_t stream, int w_dtype, int w_layout, const void* w,
                          const void* w_scale, int64_t ntaps, int64_t cin, int64_t cout,
                          void* packed);

/* Packed Q8_0 weights (spc_conv_pack_weights with SPC_Q8_0) -> packed bf16
 * weights (spc_conv_packed_bytes(SPC_BF16, ...) bytes, 16-byte aligned)
 * holding bf16(f32(d) * q) per weight: the values the Q8_0 conv feeds its
 * MFMAs, so spc_sparse_conv with (SPC_BF16, SPC_W_PACKED, packed_bf16) is
 * bit-identical to (SPC_Q8_0, SPC_W_PACKED, packed_q8).  The dequant cast
 * the reference runs before each Q8_0 conv GEMM (as_f16,
 * SRC/slat_flow_graph.cpp:24-27), as one HBM pass: a conv over many row
 * tiles (the in-register path dequantises every weight once per tile)
 * runs faster as expand + bf16 conv. */
int spc_conv_expand_q8_0(spc_stream_t stream, const void* packed_q8, int64_t ntaps, int64_t cin,
                         int64_t cout, void* packed_bf16);

/* spc_conv_expand_q8_0 with the operand type chosen: out_dtype SPC_BF16
 * (bf16(f32(d) * q), as above) or SPC_F16 (f16(f32(d) * q): exactly the
 * weights the reference's Q8_0 convs feed their f16 GEMM, as_f16 in
 * SRC/slat_flow_graph.cpp:24-27).  With f16 features (spc_convert turns
 * bf16 features into f16 exactly, inside f16's range) the f16 conv over
 * these panels takes the reference's GEMM operands. */
int spc_conv_expand_q8_0_to(spc_stream_t stream, const void* packed_q8, int64_t ntaps,
                            int64_t cin, int64_t cout, int out_dtype, void* packed_out);

/* Element conversion of n values between SPC_F32, SPC_F16 and SPC_BF16
 * (round to nearest even; bf16 -> f16 is exact for magnitudes in
 * [2^-17, 65504]).  No reference counterpart: the feature casts around
 * the f16-operand Q8_0 conv (the reference graph's ggml_cast nodes). */
int spc_convert(spc_stream_t stream, int src_dtype, const void* src, int dst_dtype, void* dst,
                int64_t n);

/* Drop-in for the reference's spconv bridge (same name, arguments and
 * layouts as cpp_ggml/third_party/sam3d-spconv/include/
 * sam3d_spconv_bridge.cuh:10-21, called from PATCH:2033-2038): f16
 * input [tokens, channels], weight [output_channels, 27, channels], bias
 * [output_channels], output [tokens, output_channels]; indices offset-major
 * [27, tokens] (-1 = missing), mask / mask_argsort the sorted masks and
 * permutation of spc_map_build, accepted and not needed: rows run in
 * natural order, which keeps each tile's gathered rows spatially coherent
 * (the output is the same in any order).  Accumulates in F32 (the
 * reference kernel accumulates in f16).  channels and output_channels must
 * be multiples of 8, as the reference's spconv iterators take them
 * (.../inpitera/ForwardDgradSparseIOIterator.h:58-61); widths that are not
 * multiples of 32 run zero-padded to the next multiple of 32 (the input
 * rows copied in, the output rows copied out; input and output 16-byte
 * aligned).  The KRSC weights are packed on every call into a
 * library-owned device buffer and the packed conv runs on them.  The tile
 * setup comes from library-owned tile plans, up to four per device keyed
 * by (tokens, tile geometry) with the least recently used replaced, each
 * with a copy of the indices it was built from (about 160 bytes per token):
 * each call checks its indices against the copy in the same launch as the
 * weight pack, and tiles whose entries changed set themselves up and
 * refresh their plan, so repeated calls over one index table skip the
 * setup, also when calls alternate between token counts.  These buffers
 * (one set per device) are grown with hipMalloc when a call needs more and
 * held until the process ends; bridge calls on one device share them, so
 * calls on different streams of one device must not overlap (the
 * reference's bridge, too, assumes one stream).  Returns nothing, like the
 * reference: spc_last_error() is cleared on entry and is non-empty after
 * the call exactly when it failed (output unwritten). */
void sam3d_spconv_f16_forward(spc_stream_t stream, const void* input, const void* weight,
                              const void* bias, void* output, const int32_t* indices,
                              const uint32_t* mask, const int32_t* mask_argsort, int64_t tokens,
                              int64_t channels, int64_t output_channels);

/* Q8_0 weights.  ggml block = [fp16 d][int8 q[32]] (34 bytes), as written by
 * quantize_q8_0 (cpp_ggml/scripts/gguf_schema.py:14-24).  Splits nblocks
 * blocks into quants qs[nblocks*32] and scales d[nblocks] (16-byte
 * aligned streams for the GEMM's in-register dequantisation). */
int spc_q8_0_repack(spc_stream_t stream, const uint8_t* blocks, int64_t nblocks, int8_t* qs,
                    uint16_t* d);

/* quantize_q8_0 (cpp_ggml/scripts/gguf_schema.py:14-24) on the GPU: n
 * floats (n % 32 == 0) -> n/32 blocks of 34 bytes.  Per block d =
 * fp16(amax / 127) (amax 0 -> 1e-12), q = clip(rint(w / f32(d)), -127, 127)
 * with rint rounding half to even.  Bit-exact with the converter. */
int spc_q8_0_quantize(spc_stream_t stream, const float* w, int64_t n, uint8_t* blocks);

/* Q8_0 blocks -> f32(d) * q in out_dtype (SPC_F32, SPC_F16 or SPC_BF16):
 * the reference's as_f32 / as_f16 dequantisation (SRC/slat_flow_graph.cpp:
 * 24-27; SRC/mesh_decoder_graph.cpp:309-312). */
int spc_q8_0_dequant(spc_stream_t stream, const uint8_t* blocks, int64_t nblocks, int out_dtype,
                     void* out);

/* ------------------------------------------------------------------------
 * Scatter-mean.  Replaces ggml_sam3d_sparse_scatter_mean (PATCH:59-63,
 * CPU semantics PATCH:151-215): out[r] = (sum over fine rows i with
 * rows[i] == r, ascending i, partial sums rounded to the storage dtype
 * after every add) / counts[r] in F32; rows outside [0, nc) skipped.
 * Deterministic (the reference CUDA kernel uses atomics, PATCH:1847-1901).
 * dtype SPC_F16 (the reference op), SPC_BF16 or SPC_F32.
 * ------------------------------------------------------------------------ */
size_t spc_scatter_mean_workspace_bytes(int64_t nf, int64_t nc);
int spc_scatter_mean(spc_stream_t stream, int dtype, const void* features, const int32_t* rows,
                     const float* counts, void* out, int64_t channels, int64_t nf, int64_t nc,
                     void* workspace, size_t workspace_bytes);

/* The scatter-mean above from spc_downsample_map's children lists instead
 * of fine_to_coarse: out[r] = (children of r, ascending fine rows, summed
 * with the same per-add rounding) / counts[r] -- the same values as
 * spc_scatter_mean on the same map, without its sort or workspace.
 * children is int32 [8 * nc], each list ended by a value outside [0, nf)
 * (the map pads with nf).  No reference counterpart: SparseDownsample's
 * fast path once the map is built (the reference module re-runs its
 * scatter_reduce every call, SP/spatial.py:59-62). */
int spc_children_mean(spc_stream_t stream, int dtype, const void* features,
                      const int32_t* children, const float* counts, void* out, int64_t channels,
                      int64_t nf, int64_t nc);

/* Row gather dst[i] = src[idx[i]] (zero row when idx[i] is outside
 * [0, n_src)).  SparseUpsample's feats[idx] (SP/spatial.py:92; SRC/
 * slat_flow_graph.cpp:244-247) and SparseSubdivide's parent broadcast
 * (SP/spatial.py:123-128; SRC/mesh_decoder_graph.cpp:386-393). */
int spc_gather_rows(spc_stream_t stream, int dtype, const void* src, const int32_t* idx,
                    void* dst, int64_t n_out, int64_t n_src, int64_t channels);

/* ------------------------------------------------------------------------
 * Residual-block prologue and epilogues (SparseResBlock3d,
 * sam3d_objects/.../models/structured_latent_flow.py:61-74; native graph
 * SRC/slat_flow_graph.cpp:284-380).
 * ------------------------------------------------------------------------ */

/* Row LayerNorm then SiLU over x [n, c] in dtype (SPC_F32 / SPC_F16 /
 * SPC_BF16), as LayerNorm32 + F.silu: mean and biased variance in F32,
 * (v - mean) / sqrt(var + eps) (* gamma + beta when gamma / beta, f32 [c],
 * are given), rounded to dtype (LayerNorm32 casts back,
 * modules/norm.py:6-8), then x * sigmoid(x) in F32 of that value, rounded
 * again (silu 0 skips it).  y may be x.  c <= 2048. */
int spc_layernorm_silu(spc_stream_t stream, int dtype, const void* x, int64_t n, int64_t c,
                       const float* gamma, const float* beta, float eps, int silu, void* y);

/* The block's second activation over rows of any width c <= 2048 (a
 * multiple of 4): u = dt(LayerNorm(x; eps)) without affine (norm2),
 * m = dt(dt(u * dt(1 + scale[b])) + shift[b]), y = dt(silu(m)), b =
 * coords[4 t] the row's batch (clamped to [0, n_batch)) -- the
 * `norm2(h) * (1 + scale) + shift` and F.silu of structured_latent_flow.py:
 * 70-71 (SRC/slat_flow_graph.cpp:350-355) in one read and one write of the
 * rows.  scale / shift f32 [n_batch, c] holding dtype values, 16-byte
 * aligned.  y may be x.  The conv epilogue SPC_EPI_NORM_MOD_SILU computes
 * the same for cout 32, 64 and 128 without the extra pass. */
int spc_layernorm_mod_silu(spc_stream_t stream, int dtype, const void* x, int64_t n, int64_t c,
                           float eps, const float* scale, const float* shift,
                           const int32_t* coords, int64_t n_batch, void* y);

/* GroupNorm over each batch item's rows (SparseGroupNorm32,
 * modules/sparse/norm.py:15-55: per item, the statistics of each group of
 * c / groups channels over all of the item's rows; biased variance, eps
 * inside the square root; computed in F32 and cast back).  Rows of item b
 * are [offsets[b], offsets[b+1]) (offsets: device int64 [n_batch + 1],
 * ascending); max_rows bounds the rows of one item.
 *   spc_group_norm_stats: stats (device f32 [n_batch, groups, 2]) =
 *     (mean, 1 / sqrt(var + eps)); F64 partial sums in a fixed order
 *     (deterministic), workspace of spc_group_norm_workspace_bytes.
 *   spc_group_norm_silu: y[i] = dt(silu(dt(x[r] * a + b))) with the
 *     per-channel a = rstd * gamma, b = beta - a * mean of r's item (the
 *     fused form torch's group_norm evaluates) and r = rows[i] (rows NULL:
 *     r = i) -- the norm, SiLU and SparseSubdivide's parent gather of
 *     SparseSubdivideBlock3d's act_layers (decoder_mesh.py:69-73) in one
 *     pass; silu 0 skips the activation; gamma / beta f32 [c] or NULL.
 * c <= 1024, a multiple of 4 and of groups. */
size_t spc_group_norm_workspace_bytes(int64_t n_batch, int64_t max_rows, int64_t groups);
int spc_group_norm_stats(spc_stream_t stream, int dtype, const void* x, int64_t c, int64_t groups,
                         const int64_t* offsets, int64_t n_batch, int64_t max_rows, float eps,
                         float* stats, void* workspace, size_t workspace_bytes);
int spc_group_norm_silu(spc_stream_t stream, int dtype, const void* x, int64_t n_src, int64_t c,
                        int64_t groups, const int64_t* offsets, int64_t n_batch, const float* stats,
                        const float* gamma, const float* beta, int silu, const int32_t* rows,
                        int64_t n_out, void* y);

/* Conv epilogues, applied to the output rows before they are stored:
 *   SPC_EPI_RESIDUAL       y = dt(dt(conv + bias) + residual[t])
 *                          (`h = conv2(h); h = h + skip`, :72-73);
 *   SPC_EPI_NORM_MOD_SILU  v = dt(conv + bias); u = dt(LayerNorm(v; eps))
 *                          over the row's cout channels (no affine);
 *                          m = dt(dt(u * dt(1 + scale[b])) + shift[b]);
 *                          y = dt(silu(m)), b = coords[4 t] the row's batch
 *                          (`norm2(h) * (1 + scale) + shift`, then SiLU,
 *                          :70-71), where dt() rounds to the feature dtype.
 * residual: [n_out, cout] in dtype, or, with residual_rows set, [n_residual,
 * cout] read at row residual_rows[t] (entries outside [0, n_residual) add
 * nothing): the subdivide block adds its skip computed on the parent rows
 * (decoder_mesh.py:82).  scale / shift: f32 [n_batch, cout]
 * holding dtype values (emb_out.type(x.dtype)).  NORM_MOD_SILU needs
 * cout 32, 64 or 128 (one tile covers a whole output row); other widths
 * run the conv and then spc_layernorm_mod_silu. */
typedef enum { SPC_EPI_NONE = 0, SPC_EPI_RESIDUAL = 1, SPC_EPI_NORM_MOD_SILU = 2 } spc_epilogue_mode;
typedef struct {
    int32_t mode;
    float eps;
    const void* residual;
    const float* scale;
    const float* shift;
    const int32_t* coords;
    int64_t n_batch;
    const int32_t* residual_rows;
    int64_t n_residual;
} spc_conv_epilogue;

/* spc_sparse_conv_plan with an epilogue (epi NULL or mode SPC_EPI_NONE:
 * identical to spc_sparse_conv_plan).  No reference counterpart as one
 * call: it fuses the reference's separate conv, norm, modulation,
 * activation and residual nodes. */
int spc_sparse_conv_fused(spc_stream_t stream, int dtype, const void* x, int w_dtype,
                          int w_layout, const void* w, const void* w_scale, const void* bias,
                          void* y, const int32_t* idx, int idx_layout, const int32_t* row_perm,
                          const void* plan, int64_t ntaps, int64_t n_out, int64_t n_in,
                          int64_t cin, int64_t cout, const spc_conv_epilogue* epi);

/* spc_sparse_conv_fused with weight classes: the rows of tile order
 * [c * class_rows, (c + 1) * class_rows) (class_rows a multiple of 256)
 * use taps c * ntaps .. c * ntaps + ntaps - 1 of packed weights holding
 * n_classes * ntaps taps (spc_conv_pack_weights with that tap count, in the
 * feature dtype; no Q8_0).  n_out <= class_rows * n_classes counts tile
 * rows; with row_perm each tile row writes output row row_perm[v] (-1 =
 * none), so y holds max(row_perm) + 1 rows.  No reference counterpart (the
 * merged-tap child conv of spc_subdivide_tap_classes). */
int spc_sparse_conv_classes(spc_stream_t stream, int dtype, const void* x, const void* w,
                            const void* bias, void* y, const int32_t* idx, int idx_layout,
                            const int32_t* row_perm, const void* plan, int64_t ntaps,
                            int64_t n_out, int64_t n_in, int64_t cin, int64_t cout,
                            int64_t class_rows, int64_t n_classes, const spc_conv_epilogue* epi);

#ifdef __cplusplus
}
#endif

#endif /* SAM3D_SPCONV_AMD_H */
