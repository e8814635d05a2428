// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A C-ABI wrapper around the reference's own host table builders
// (SRC/sparse_ops.{hpp,cpp}, SRC = cpp_ggml/src of the reference).  The
// Makefile beside this file compiles it together with the reference's
// unmodified sparse_ops.cpp into oracle/_ref/libref_tables.so, which tests
// load to pin the oracle's restatement (spconv_oracle.cpp) and which
// tests/golden/make_golden.py runs to write the golden fixtures.
#include "sparse_ops.hpp"

#include <cstdint>
#include <cstring>

extern "C" {

// SlatTables::build (SRC/sparse_ops.cpp:23-186); copies out every table.
// Buffers: conv_fine / conv_fine_spconv [27*nf], mask / argsort / f2c [nf],
// conv_coarse / conv_coarse_spconv [27*nf] (upper bound), coarse mask /
// argsort / count [nf], coarse_children [8*nf].  Returns nc, or -1.
int64_t ref_slat_tables(const int32_t* coords, int64_t nf, int32_t* conv_fine,
                        int32_t* conv_fine_spconv, int32_t* fine_mask, int32_t* fine_argsort,
                        int32_t* fine_to_coarse, int32_t* coarse_children, float* coarse_count,
                        int32_t* conv_coarse, int32_t* conv_coarse_spconv, int32_t* coarse_mask,
                        int32_t* coarse_argsort) {
    sam3d::SlatTables t;
    // channels=6 keeps the (unrelated) positional-embedding table small
    if (!t.build(coords, nf, 6)) return -1;
    auto put = [](const std::vector<int32_t>& v, int32_t* dst) {
        if (dst) std::memcpy(dst, v.data(), v.size() * sizeof(int32_t));
    };
    put(t.conv_fine, conv_fine);
    put(t.conv_fine_spconv, conv_fine_spconv);
    put(t.conv_fine_mask, fine_mask);
    put(t.conv_fine_argsort, fine_argsort);
    put(t.fine_to_coarse, fine_to_coarse);
    put(t.coarse_children, coarse_children);
    if (coarse_count)
        std::memcpy(coarse_count, t.coarse_count.data(), t.coarse_count.size() * sizeof(float));
    put(t.conv_coarse, conv_coarse);
    put(t.conv_coarse_spconv, conv_coarse_spconv);
    put(t.conv_coarse_mask, coarse_mask);
    put(t.conv_coarse_argsort, coarse_argsort);
    return t.nc;
}

// MeshTables::build (SRC/sparse_ops.cpp:375-391): three levels.  Returns 1 on
// success, 0 on failure; level sizes are written to sizes[3].  Coordinate
// and conv buffers may be null (sizes only) and are sized by the caller
// from a first call.
int ref_mesh_tables(const int32_t* coords, int64_t n, int base_resolution, int64_t* sizes,
                    int32_t* coords1, int32_t* coords2, int32_t* conv0, int32_t* conv1,
                    int32_t* conv2) {
    sam3d::MeshTables t;
    if (!t.build(coords, n, base_resolution)) return 0;
    for (int l = 0; l < 3; ++l) sizes[l] = t.levels[l].n;
    auto put = [](const std::vector<int32_t>& v, int32_t* dst) {
        if (dst) std::memcpy(dst, v.data(), v.size() * sizeof(int32_t));
    };
    put(t.levels[1].coords, coords1);
    put(t.levels[2].coords, coords2);
    put(t.levels[0].conv, conv0);
    put(t.levels[1].conv, conv1);
    put(t.levels[2].conv, conv2);
    return 1;
}

}  // extern "C"
