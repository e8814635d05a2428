// maps.hip -- kernel-map construction on the GPU.
//
//   spc_map_build       : submanifold 3x3x3 neighbour tables (SlatTables::
//                         build's conv tables, SRC/sparse_ops.cpp:93-155, and
//                         build_mesh_conv_table, SRC/sparse_ops.cpp:312-346)
//   spc_downsample_map  : stride-2 coarse map (SRC/sparse_ops.cpp:27-81)
//   spc_subdivide_map   : 2x subdivision (SRC/sparse_ops.cpp:348-371)
//
// Design: an open-addressing hash table in HBM (power-of-two capacity >= 2N,
// 64-bit packed (b,x,y,z) keys, linear probing, atomicCAS insert, atomicMin
// of the row id so the first occurrence of a duplicate owns the key exactly
// like std::map::emplace).  The 27-offset query runs one workgroup per 64
// tokens: 27x64 probes land in LDS, then the token-major table, the
// offset-major table (27 coalesced 256-byte rows) and the masks are written
// from LDS with unit-stride stores.  The stable mask argsort is the radix
// sort of sort.hip.
#include <climits>

#include <algorithm>
#include <atomic>

#include "common.h"

namespace spc {

namespace {

enum : int32_t { kErrBadCoord = 1, kErrDup = 2, kErrOom = 4 };

__device__ inline bool coord_ok(int4 c, int32_t lim) {
    return c.x >= 0 && c.x < kBatchLimit && c.y >= 0 && c.y < lim && c.z >= 0 && c.z < lim &&
           c.w >= 0 && c.w < lim;
}

__global__ void map_init_kernel(unsigned long long* hkeys, int32_t* hvals, int64_t cap,
                                int32_t* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < cap) {
        hkeys[i] = kEmptyKey;
        hvals[i] = INT_MAX;
    }
    if (i == 0) *status = 0;
}

__global__ __launch_bounds__(256) void hash_insert_kernel(const int4* __restrict__ coords,
                                                          int64_t n, int32_t lim,
                                                          unsigned long long* hkeys,
                                                          int32_t* hvals, uint32_t cap_mask,
                                                          int32_t* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int4 c = coords[i];
    if (!coord_ok(c, lim)) {
        atomicOr(status, kErrBadCoord);
        return;
    }
    const unsigned long long key = pack_key(c.x, c.y, c.z, c.w);
    uint32_t h = hash_key(key) & cap_mask;
    for (uint32_t it = 0; it <= cap_mask; ++it) {
        const unsigned long long prev = atomicCAS(&hkeys[h], kEmptyKey, key);
        if (prev == kEmptyKey || prev == key) {
            atomicMin(&hvals[h], (int32_t)i);
            return;
        }
        h = (h + 1) & cap_mask;
    }
    atomicOr(status, kErrOom);
}

// Dense grid: every cell INT_MAX, then each row takes its cell by atomicMin
// (the first row of a duplicated coordinate owns it, like the hash table).
__global__ void dense_init_kernel(int32_t* __restrict__ grid, int64_t cells4, int32_t* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < cells4) reinterpret_cast<int4*>(grid)[i] = int4{INT_MAX, INT_MAX, INT_MAX, INT_MAX};
    if (i == 0) *status = 0;
}

__global__ __launch_bounds__(256) void dense_insert_kernel(const int4* __restrict__ coords,
                                                           int64_t n, int32_t n_batch, int32_t res,
                                                           int32_t* grid, int32_t* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int4 c = coords[i];
    if (c.x < 0 || c.x >= n_batch || c.y < 0 || c.y >= res || c.z < 0 || c.z >= res || c.w < 0 ||
        c.w >= res) {
        atomicOr(status, kErrBadCoord);
        return;
    }
    atomicMin(&grid[(((int64_t)c.x * res + c.y) * res + c.z) * res + c.w], (int32_t)i);
}

// Row lookups of the 27-offset query: the hash table, or a dense grid
// [n_batch][R][R][R] of row ids when the caller bounds the coordinates.
// kTokens: rows per 256-thread block of the query.  Hash probes chain
// dependent loads, so more, smaller blocks hide them better (4 ellipsoid
// shells, 62,710 rows: 64 -> 16 rows per block, hash build 101 -> 86 us);
// the dense grid's single loads favour 32 (dense build 53.5 -> 53.0 us).
// A lookup runs in three steps so that a thread's lookups can have their
// memory loads in flight together: start (the key and its first slot, or
// dead), first (the one load most lookups need) and finish (the value;
// the hash table's rare continued probe).
struct HashLookup {
    static constexpr int kTokens = 16;
    const unsigned long long* hkeys;
    const int32_t* hvals;
    uint32_t cap_mask;
    struct Probe {
        unsigned long long key;
        uint32_t h;
        bool live;
    };
    __device__ Probe start(int b, int x, int y, int z) const {
        Probe p{0ull, 0u, false};
        if (b < 0 || b >= kBatchLimit || x < 0 || x >= kCoordLimit || y < 0 || y >= kCoordLimit ||
            z < 0 || z >= kCoordLimit)
            return p;
        p.key = pack_key(b, x, y, z);
        p.h = hash_key(p.key) & cap_mask;
        p.live = true;
        return p;
    }
    __device__ unsigned long long first(const Probe& p) const { return p.live ? hkeys[p.h] : kEmptyKey; }
    __device__ int32_t finish(const Probe& p, unsigned long long k) const {
        if (!p.live || k == kEmptyKey) return -1;
        if (k == p.key) return hvals[p.h];
        // collision at the first slot: probe on from the next one
        uint32_t h = (p.h + 1) & cap_mask;
        for (uint32_t it = 0; it < cap_mask; ++it) {
            const unsigned long long kk = hkeys[h];
            if (kk == p.key) return hvals[h];
            if (kk == kEmptyKey) return -1;
            h = (h + 1) & cap_mask;
        }
        return -1;
    }
};

struct DenseLookup {
    static constexpr int kTokens = 32;
    const int32_t* grid;
    int32_t n_batch;
    int32_t res;
    struct Probe {
        int64_t cell;  // -1: outside the grid
    };
    __device__ Probe start(int b, int x, int y, int z) const {
        if (b < 0 || b >= n_batch || x < 0 || x >= res || y < 0 || y >= res || z < 0 || z >= res)
            return Probe{-1};
        return Probe{(((int64_t)b * res + x) * res + y) * res + z};
    }
    __device__ int32_t first(const Probe& p) const { return p.cell >= 0 ? grid[p.cell] : INT_MAX; }
    __device__ int32_t finish(const Probe&, int32_t v) const { return v == INT_MAX ? -1 : v; }
};

// MESH: duplicates are an error (build_mesh_conv_table); otherwise the
// SlatTables rule applies (only the owning row gets its neighbours).
template <bool MESH, typename Lookup>
__global__ __launch_bounds__(256) void neighbor_kernel(
    const int4* __restrict__ coords, int64_t n, Lookup find, int32_t* __restrict__ token_major,
    int32_t* __restrict__ offset_major, int32_t* __restrict__ mask_nat, int32_t* status) {
    __shared__ int32_t nb[27][Lookup::kTokens + 1];
    __shared__ int32_t owner[Lookup::kTokens];
    const int tid = threadIdx.x;
    const int64_t t0 = (int64_t)blockIdx.x * Lookup::kTokens;
    // the thread's (offset, token) pairs e = tid + 256 i: every lookup's
    // first load issued before any result is needed
    constexpr int PER = (27 * Lookup::kTokens + 255) / 256;
    typename Lookup::Probe pr[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = tid + 256 * i;
        const int o = e / Lookup::kTokens;
        const int tl = e % Lookup::kTokens;
        const int64_t t = t0 + tl;
        if (e < 27 * Lookup::kTokens && t < n) {
            const int4 c = coords[t];
            pr[i] = find.start(c.x, c.y + (o / 9 - 1), c.z + ((o / 3) % 3 - 1), c.w + (o % 3 - 1));
        } else {
            pr[i] = find.start(-1, 0, 0, 0);  // dead
        }
    }
    decltype(find.first(pr[0])) fk[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) fk[i] = find.first(pr[i]);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = tid + 256 * i;
        if (e < 27 * Lookup::kTokens) nb[e / Lookup::kTokens][e % Lookup::kTokens] = find.finish(pr[i], fk[i]);
    }
    __syncthreads();
    if (tid < Lookup::kTokens) {
        const int64_t t = t0 + tid;
        int own = 0;
        if (t < n) {
            own = nb[13][tid] == (int32_t)t;
            if (MESH && !own) atomicOr(status, kErrDup);
        }
        owner[tid] = own;
    }
    __syncthreads();
    const int64_t valid_tokens = n - t0 < Lookup::kTokens ? n - t0 : Lookup::kTokens;
    if (token_major) {
        for (int e = tid; e < 27 * valid_tokens; e += 256) {
            const int tl = e / 27;
            const int o = e % 27;
            const int32_t v = owner[tl] ? nb[o][tl] : -1;
            token_major[t0 * 27 + e] = v >= 0 ? v : (int32_t)n;
        }
    }
    if (offset_major) {
        for (int e = tid; e < 27 * Lookup::kTokens; e += 256) {
            const int o = e / Lookup::kTokens;
            const int tl = e % Lookup::kTokens;
            if (tl < valid_tokens) {
                const int32_t v = owner[tl] ? nb[o][tl] : -1;
                offset_major[(int64_t)o * n + t0 + tl] = v;
            }
        }
    }
    if (mask_nat && tid < valid_tokens) {
        int32_t m = 0;
        if (owner[tid]) {
#pragma unroll
            for (int o = 0; o < 27; ++o) m |= (nb[o][tid] >= 0 ? 1 : 0) << o;
        }
        mask_nat[t0 + tid] = m;
    }
}

int status_to_code(int32_t bits) {
    if (bits & kErrBadCoord) return SPC_BAD_COORD;
    if (bits & kErrDup) return SPC_DUP_COORD;
    if (bits & kErrOom) return SPC_OOM;
    return SPC_OK;
}

int read_status_word(hipStream_t s, int32_t* dev) {
    int32_t bits = 0;
    SPC_HIP(hipMemcpyAsync(&bits, dev, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    SPC_HIP(hipStreamSynchronize(s));
    const int code = status_to_code(bits);
    if (code != SPC_OK) set_last_error("device reported: %s", spc_status_string(code));
    return code;
}

int64_t hash_capacity(int64_t n) {
    int64_t cap = 256;
    while (cap < 2 * n) cap <<= 1;
    return cap;
}

struct MapWs {
    int32_t* status;
    unsigned long long* hkeys;
    int32_t* hvals;
    int32_t* mask_nat;
    uint32_t* mask_sorted;
    int32_t* argsort;
    void* sort_ws;
    size_t sort_bytes;
};

template <typename C>
void carve_map_ws(C& c, int64_t n, MapWs* w) {
    const int64_t cap = hash_capacity(n);
    auto* st = c.template take<int32_t>(kStatusBytes / 4);
    auto* hk = c.template take<unsigned long long>(cap);
    auto* hv = c.template take<int32_t>(cap);
    auto* mn = c.template take<int32_t>(n);
    auto* ms = c.template take<uint32_t>(n);
    auto* ar = c.template take<int32_t>(n);
    const size_t sb = radix_sort_ws_bytes(n, 4);
    auto* sw = c.template take<char>(sb);
    if (w) *w = MapWs{st, hk, hv, mn, ms, ar, sw, sb};
}

// dense grid workspace: status, grid [n_batch * R^3] (a multiple of 4 cells),
// then the same mask / sort buffers
template <typename C>
void carve_dense_ws(C& c, int64_t n, int64_t cells, MapWs* w, int32_t** grid) {
    auto* st = c.template take<int32_t>(kStatusBytes / 4);
    auto* g = c.template take<int32_t>((size_t)((cells + 3) / 4 * 4));
    auto* mn = c.template take<int32_t>(n);
    auto* ms = c.template take<uint32_t>(n);
    auto* ar = c.template take<int32_t>(n);
    const size_t sb = radix_sort_ws_bytes(n, 4);
    auto* sw = c.template take<char>(sb);
    if (w) *w = MapWs{st, nullptr, nullptr, mn, ms, ar, sw, sb};
    if (grid) *grid = g;
}

// the 27-offset query, the masks' stable sort and the optional status read
// shared by the hash and the dense builds
template <typename Lookup>
int finish_map(hipStream_t s, const int4* c4, int64_t n, bool mesh, Lookup find, uint32_t flags,
               int32_t* token_major, int32_t* offset_major, int32_t* mask_sorted, int32_t* argsort,
               int32_t* mask_natural, const MapWs& w) {
    int32_t* mnat = mask_natural ? mask_natural : w.mask_nat;
    const unsigned nb = (unsigned)((n + Lookup::kTokens - 1) / Lookup::kTokens);
    if (mesh)
        neighbor_kernel<true, Lookup><<<nb, 256, 0, s>>>(c4, n, find, token_major, offset_major,
                                                         mnat, w.status);
    else
        neighbor_kernel<false, Lookup><<<nb, 256, 0, s>>>(c4, n, find, token_major, offset_major,
                                                          mnat, w.status);
    SPC_HIP(hipGetLastError());
    if (mask_sorted || argsort) {
        uint32_t* ms = mask_sorted ? reinterpret_cast<uint32_t*>(mask_sorted) : w.mask_sorted;
        int32_t* ar = argsort ? argsort : w.argsort;
        SPC_HIP(radix_sort_u32(s, reinterpret_cast<const uint32_t*>(mnat), nullptr, ms, ar, n, 27,
                               w.sort_ws, w.sort_bytes));
    }
    if (flags & SPC_MAP_SYNC) return read_status_word(s, w.status);
    return SPC_OK;
}

// ---- downsample ---------------------------------------------------------

__global__ void coarse_key_kernel(const int4* __restrict__ coords, int64_t nf, int64_t n_batch,
                                  int32_t res, int cbits, unsigned long long* __restrict__ keys,
                                  int32_t* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nf) return;
    const int4 c = coords[i];
    if (c.x < 0 || c.x >= n_batch || c.y < 0 || c.y >= res || c.z < 0 || c.z >= res || c.w < 0 ||
        c.w >= res) {
        atomicOr(status, kErrBadCoord);
        keys[i] = 0;
        return;
    }
    // (b, x/2, y/2, z/2), most significant first: lexicographic order
    keys[i] = ((unsigned long long)c.x << (3 * cbits)) |
              ((unsigned long long)(c.y >> 1) << (2 * cbits)) |
              ((unsigned long long)(c.z >> 1) << cbits) | (unsigned long long)(c.w >> 1);
}

__global__ void head_flag_kernel(const unsigned long long* __restrict__ sk, int64_t n,
                                 int32_t* __restrict__ flag) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p < n) flag[p] = (p == 0 || sk[p] != sk[p - 1]) ? 1 : 0;
}

__global__ void downsample_assign_kernel(const unsigned long long* __restrict__ sk,
                                         const int32_t* __restrict__ sv,
                                         const int32_t* __restrict__ flag,
                                         const int32_t* __restrict__ excl, int64_t nf, int cbits,
                                         int32_t* __restrict__ fine_to_coarse,
                                         int32_t* __restrict__ head_pos,
                                         int4* __restrict__ coarse_coords) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= nf) return;
    const int32_t id = excl[p] + flag[p] - 1;
    fine_to_coarse[sv[p]] = id;
    if (flag[p]) {
        head_pos[id] = (int32_t)p;
        const unsigned long long k = sk[p];
        const unsigned long long m = (1ull << cbits) - 1ull;
        coarse_coords[id] = make_int4((int32_t)(k >> (3 * cbits)), (int32_t)((k >> (2 * cbits)) & m),
                                      (int32_t)((k >> cbits) & m), (int32_t)(k & m));
    }
    if (p == nf - 1) head_pos[id + 1] = (int32_t)nf;
}

__global__ void downsample_children_kernel(const int32_t* __restrict__ sv,
                                           const int32_t* __restrict__ head_pos,
                                           const int32_t* __restrict__ nc_dev,
                                           const int4* __restrict__ coords, int64_t nf,
                                           int32_t* __restrict__ children,
                                           float* __restrict__ counts,
                                           int32_t* __restrict__ taps, int32_t* status) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= *nc_dev) return;
    const int32_t h = head_pos[id];
    const int32_t run = head_pos[id + 1] - h;
    for (int j = 0; j < 8; ++j) children[id * 8 + j] = j < run ? sv[h + j] : (int32_t)nf;
    counts[id] = (float)(run + 1);
    if (taps) {
        int32_t t[8];
        for (int j = 0; j < 8; ++j) t[j] = (int32_t)nf;
        bool dup = false;
        for (int j = 0; j < run; ++j) {
            const int32_t f = sv[h + j];
            const int4 c = coords[f];
            const int k = (c.y & 1) * 4 + (c.z & 1) * 2 + (c.w & 1);
            if (t[k] != (int32_t)nf) dup = true;
            t[k] = f;
        }
        if (dup) atomicOr(status, kErrDup);
        for (int j = 0; j < 8; ++j) taps[id * 8 + j] = t[j];
    }
}

int bits_for(int64_t v) {  // bits needed to hold values in [0, v)
    int b = 0;
    while (b < 62 && (1ll << b) < v) ++b;
    return b;
}

// ---- subdivide ------------------------------------------------------------

// Transposed stride-2 map: fine row f reads coarse row fine_to_coarse[f] at
// its own tap k(f) = (x&1)*4 + (y&1)*2 + (z&1); every other tap is nc.
__global__ void stride2_inverse_kernel(const int4* __restrict__ coords,
                                       const int32_t* __restrict__ f2c, int64_t nf, int32_t nc,
                                       int32_t* __restrict__ taps) {
    const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nf) return;
    const int4 c = coords[f];
    const int k = (c.y & 1) * 4 + (c.z & 1) * 2 + (c.w & 1);
    const int32_t p = f2c[f];
    int32_t t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = j == k ? p : nc;
    int4* dst = reinterpret_cast<int4*>(taps + f * 8);
    dst[0] = int4{t[0], t[1], t[2], t[3]};
    dst[1] = int4{t[4], t[5], t[6], t[7]};
}

__global__ void subdivide_flag_kernel(const uint8_t* __restrict__ keep, int64_t m8,
                                      int32_t* __restrict__ flag) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < m8) flag[i] = keep[i] ? 1 : 0;
}

__global__ void subdivide_kernel(const int4* __restrict__ coords, int64_t n,
                                 const uint8_t* __restrict__ keep,
                                 const int32_t* __restrict__ pos, int4* __restrict__ out_coords,
                                 int32_t* __restrict__ parent, int32_t* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * 8) return;
    if (keep && !keep[i]) return;
    const int64_t p = i >> 3;
    const int c = (int)(i & 7);
    const int4 s = coords[p];
    if (s.x < 0 || s.x >= kBatchLimit || s.y < 0 || s.z < 0 || s.w < 0 ||
        s.y >= kCoordLimit / 2 || s.z >= kCoordLimit / 2 || s.w >= kCoordLimit / 2)
        atomicOr(status, kErrBadCoord);
    const int64_t dst = keep ? pos[i] : i;
    out_coords[dst] = make_int4(s.x, s.y * 2 + c / 4, s.z * 2 + (c / 2) % 2, s.w * 2 + c % 2);
    parent[dst] = (int32_t)p;
}

// out[i] = rows[idx[i]] for idx[i] in [0, n_rows), else -1; four entries per
// lane (n4 = n / 4 vector steps, then the tail)
__global__ void compose_rows_kernel(const int32_t* __restrict__ idx, int64_t n,
                                    const int32_t* __restrict__ rows, int64_t n_rows,
                                    int32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n4 = n / 4;
    auto one = [&](int32_t v) { return (v >= 0 && v < n_rows) ? rows[v] : -1; };
    if (i < n4) {
        const int4 v = reinterpret_cast<const int4*>(idx)[i];
        reinterpret_cast<int4*>(out)[i] = int4{one(v.x), one(v.y), one(v.z), one(v.w)};
    } else if (i - n4 < n - 4 * n4) {
        const int64_t j = 4 * n4 + (i - n4);
        out[j] = one(idx[j]);
    }
}

// Child table of a fully subdivided tensor from the parents' table: child
// c = 8p + d (d = dx*4 + dy*2 + dz) at 2*x_p + d; its neighbour at offset
// delta(o) is child e of parent p + j, per axis s = d + delta, j = floor(s/2),
// e = s - 2j.  Non-owning (duplicate) parents give children with no
// neighbours, as the hash table's first-row rule gives for their copies.
// A block takes kSnParents parents: their table rows are read once into LDS
// (coalesced), then the block's 8 * 27 entries per parent are written in
// order (coalesced).  The host bounds 8 * np * 27 by INT32_MAX.
constexpr int kSnParents = 32;

__global__ __launch_bounds__(256) void subdivide_neighbors_kernel(const int32_t* __restrict__ ptm,
                                                                  int64_t np,
                                                                  int32_t* __restrict__ ctm) {
    __shared__ int32_t pt[kSnParents * 27];
    const uint32_t p0 = blockIdx.x * kSnParents;
    const uint32_t npb = min((uint32_t)kSnParents, (uint32_t)np - p0);
    for (uint32_t k = threadIdx.x; k < npb * 27u; k += blockDim.x) pt[k] = ptm[(size_t)p0 * 27 + k];
    __syncthreads();
    const uint32_t nc = 8u * (uint32_t)np;
    const uint32_t base = p0 * 8u * 27u;
    for (uint32_t k = threadIdx.x; k < npb * 8u * 27u; k += blockDim.x) {
        const uint32_t cl = k / 27u;         // child within the block
        const int o = (int)(k - cl * 27u);
        const uint32_t pl = cl >> 3;         // parent within the block
        const int d = (int)(cl & 7u);
        const int32_t* pr = pt + pl * 27u;
        int32_t out = (int32_t)nc;
        if (pr[13] == (int32_t)(p0 + pl)) {
            const int sx = (d >> 2) + o / 9 - 1, sy = ((d >> 1) & 1) + (o / 3) % 3 - 1,
                      sz = (d & 1) + o % 3 - 1;
            const int jx = sx >> 1, jy = sy >> 1, jz = sz >> 1;  // floor division (arithmetic shift)
            const int q = pr[(jx + 1) * 9 + (jy + 1) * 3 + (jz + 1)];
            if (q >= 0 && q < np)
                out = q * 8 + (sx - 2 * jx) * 4 + (sy - 2 * jy) * 2 + (sz - 2 * jz);
        }
        ctm[base + k] = out;
    }
}

// Merged-tap tables of the 3x3x3 conv over a fully subdivided tensor, read
// from the parents.  Child c = 8p + d sees, per axis, parent offsets
// {d_a - 1, d_a}: tap t = ix*4 + iy*2 + iz at j_a = d_a - 1 + i_a.
// idx[c*8 + t] = the parent row at x_p + j (or -1); perm is class-major:
// perm[d*class_rows + i] = 8i + d for i < np, -1 for the padding rows.
__global__ __launch_bounds__(256) void subdivide_tap_classes_kernel(const int32_t* __restrict__ ptm,
                                                                    int64_t np, int64_t class_rows,
                                                                    int32_t* __restrict__ idx,
                                                                    int32_t* __restrict__ perm) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < 64 * np) {
        const int64_t c = e >> 3;
        const int t = (int)(e & 7);
        const int64_t p = c >> 3;
        const int d = (int)(c & 7);
        const int32_t* pr = ptm + p * 27;
        int32_t out = -1;
        if (pr[13] == (int32_t)p) {  // a duplicate parent's children have no neighbours
            const int jx = (d >> 2) - 1 + (t >> 2), jy = ((d >> 1) & 1) - 1 + ((t >> 1) & 1),
                      jz = (d & 1) - 1 + (t & 1);
            const int32_t q = pr[(jx + 1) * 9 + (jy + 1) * 3 + (jz + 1)];
            if (q >= 0 && q < np) out = q;
        }
        idx[e] = out;
    }
    if (e < 8 * class_rows) {
        const int64_t d = e / class_rows;
        const int64_t i = e - d * class_rows;
        perm[e] = i < np ? (int32_t)(8 * i + d) : -1;
    }
}

inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---- the map build's scratch for callers that cannot allocate ------------
// (spc_map_build_noalloc).  One 56 MiB array per device, held until the
// process ends: the hash-table map workspace of up to kNoAllocMaxN voxels
// (spc_map_workspace_bytes(2^20) is about 53 MiB).  Every call on a device
// shares it; the build's init kernel rewrites everything the build reads
// (hash slots, status word) before use, so nothing carries over between
// calls, but calls that overlap on one device race.
constexpr int64_t kNoAllocMaxN = (int64_t)1 << 20;
constexpr size_t kScratchBytes = (size_t)56 << 20;
__device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device with that device current.  In host code `scratch` is a stand-in
// symbol, not a device address: kernels and copies get this pointer only.
void* scratch_addr() {
    static std::atomic<void*> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    void* p = cache[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_last_error("spc_map_build_noalloc: hipGetSymbolAddress(scratch) failed on "
                           "device %d: %s", dev, hipGetErrorString(e));
            return nullptr;
        }
        cache[dev].store(p, std::memory_order_release);
    }
    return p;
}

}  // namespace
}  // namespace spc

using namespace spc;

extern "C" {

size_t spc_map_workspace_bytes(int64_t n) {
    Sizer z;
    carve_map_ws(z, n > 0 ? n : 1, nullptr);
    return z.used + 256;
}

int spc_map_build(spc_stream_t stream, const int32_t* coords, int64_t n, int32_t resolution,
                  uint32_t flags, int32_t* token_major, int32_t* offset_major,
                  int32_t* mask_sorted, int32_t* argsort, int32_t* mask_natural,
                  void* workspace, size_t workspace_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n <= 0 || n > INT32_MAX / 27) {
        set_last_error("spc_map_build: n = %lld out of range", (long long)n);
        return SPC_BAD_SHAPE;
    }
    if (!coords || !workspace || !aligned16(coords)) {
        set_last_error("spc_map_build: null or misaligned coords / workspace");
        return SPC_BAD_ARG;
    }
    const bool mesh = flags & SPC_MAP_MESH;
    if (mesh && (resolution <= 0 || resolution > kCoordLimit)) {
        set_last_error("spc_map_build: resolution %d outside (0, %d]", resolution, kCoordLimit);
        return SPC_BAD_ARG;
    }
    Carver c(workspace, workspace_bytes);
    MapWs w;
    carve_map_ws(c, n, &w);
    if (!c.ok) {
        set_last_error("spc_map_build: workspace of %zu bytes < %zu", workspace_bytes,
                       spc_map_workspace_bytes(n));
        return SPC_OOM;
    }
    const int64_t cap = hash_capacity(n);
    const uint32_t cap_mask = (uint32_t)(cap - 1);
    const int4* c4 = reinterpret_cast<const int4*>(coords);
    map_init_kernel<<<grid_for(cap, 256), 256, 0, s>>>(w.hkeys, w.hvals, cap, w.status);
    hash_insert_kernel<<<grid_for(n, 256), 256, 0, s>>>(c4, n, mesh ? resolution : kCoordLimit,
                                                        w.hkeys, w.hvals, cap_mask, w.status);
    return finish_map(s, c4, n, mesh, HashLookup{w.hkeys, w.hvals, cap_mask}, flags, token_major,
                      offset_major, mask_sorted, argsort, mask_natural, w);
}

int spc_map_build_noalloc(spc_stream_t stream, const int32_t* coords, int64_t n,
                          int32_t resolution, uint32_t flags, int32_t* token_major,
                          int32_t* offset_major, int32_t* mask_sorted, int32_t* argsort,
                          int32_t* mask_natural) {
    if (n > kNoAllocMaxN || spc_map_workspace_bytes(n) > kScratchBytes) {
        set_last_error("spc_map_build_noalloc: n = %lld above the maximum %lld of the library's "
                       "static scratch (use spc_map_build with a workspace)", (long long)n,
                       (long long)kNoAllocMaxN);
        return SPC_BAD_SHAPE;
    }
    void* ws = scratch_addr();
    if (ws == nullptr) return SPC_HIP_ERROR;
    return spc_map_build(stream, coords, n, resolution, flags, token_major, offset_major,
                         mask_sorted, argsort, mask_natural, ws, kScratchBytes);
}

// n_batch * resolution^3 within 2^32 cells, tested by division: the product
// itself reaches 2^63 at the domain's ends (2^18 batches of 32768^3)
static bool dense_cells_ok(int64_t n_batch, int32_t resolution) {
    if (n_batch <= 0 || n_batch > kBatchLimit || resolution <= 0 || resolution > kCoordLimit)
        return false;
    const int64_t r = resolution;
    return n_batch <= ((int64_t)1 << 32) / (r * r * r);
}

size_t spc_map_dense_workspace_bytes(int64_t n, int64_t n_batch, int32_t resolution) {
    if (!dense_cells_ok(n_batch, resolution)) return 0;
    const int64_t r = resolution;
    Sizer z;
    carve_dense_ws(z, n > 0 ? n : 1, n_batch * r * r * r, nullptr, nullptr);
    return z.used + 256;
}

int spc_map_build_dense(spc_stream_t stream, const int32_t* coords, int64_t n, int64_t n_batch,
                        int32_t resolution, uint32_t flags, int32_t* token_major,
                        int32_t* offset_major, int32_t* mask_sorted, int32_t* argsort,
                        int32_t* mask_natural, void* workspace, size_t workspace_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n <= 0 || n > INT32_MAX / 27 || !dense_cells_ok(n_batch, resolution)) {
        set_last_error("spc_map_build_dense: n = %lld, n_batch = %lld, resolution = %d out of range "
                       "(at most 2^32 cells)", (long long)n, (long long)n_batch, resolution);
        return SPC_BAD_SHAPE;
    }
    if (!coords || !workspace || !aligned16(coords)) {
        set_last_error("spc_map_build_dense: null or misaligned coords / workspace");
        return SPC_BAD_ARG;
    }
    const int64_t r = resolution;
    const int64_t cells = n_batch * r * r * r;
    Carver c(workspace, workspace_bytes);
    MapWs w;
    int32_t* grid = nullptr;
    carve_dense_ws(c, n, cells, &w, &grid);
    if (!c.ok) {
        set_last_error("spc_map_build_dense: workspace of %zu bytes < %zu", workspace_bytes,
                       spc_map_dense_workspace_bytes(n, n_batch, resolution));
        return SPC_OOM;
    }
    const int4* c4 = reinterpret_cast<const int4*>(coords);
    const int64_t cells4 = (cells + 3) / 4;
    dense_init_kernel<<<grid_for(cells4, 256), 256, 0, s>>>(grid, cells4, w.status);
    dense_insert_kernel<<<grid_for(n, 256), 256, 0, s>>>(c4, n, (int32_t)n_batch, resolution, grid,
                                                         w.status);
    return finish_map(s, c4, n, (flags & SPC_MAP_MESH) != 0,
                      DenseLookup{grid, (int32_t)n_batch, resolution}, flags, token_major,
                      offset_major, mask_sorted, argsort, mask_natural, w);
}

int spc_read_status(spc_stream_t stream, void* workspace) {
    if (!workspace) return SPC_BAD_ARG;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int32_t* st = static_cast<int32_t*>(workspace);
    const int code = read_status_word(s, st);
    SPC_HIP(fill_i32(s, st, 0, 1));
    return code;
}

size_t spc_downsample_workspace_bytes(int64_t nf) {
    const int64_t n = nf > 0 ? nf : 1;
    Sizer z;
    z.take<int32_t>(kStatusBytes / 4);
    z.take<unsigned long long>(n);  // keys
    z.take<unsigned long long>(n);  // sorted keys
    z.take<int32_t>(n);             // sorted values
    z.take<int32_t>(n);             // head flags
    z.take<int32_t>(n);             // exclusive scan
    z.take<int32_t>(n + 1);         // head positions
    z.take<int32_t>(1);             // nc
    z.take<char>(radix_sort_ws_bytes(n, 8));
    z.take<char>(scan_ws_bytes(n));
    return z.used + 256;
}

int spc_downsample_map(spc_stream_t stream, const int32_t* coords, int64_t nf, int64_t n_batch,
                       int32_t resolution, int32_t* fine_to_coarse, int32_t* coarse_coords,
                       int32_t* children, float* counts, int32_t* stride2_taps,
                       int64_t* nc_out, void* workspace, size_t workspace_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (nf <= 0 || nf > INT32_MAX / 8) {
        set_last_error("spc_downsample_map: nf = %lld out of range", (long long)nf);
        return SPC_BAD_SHAPE;
    }
    if (!coords || !fine_to_coarse || !coarse_coords || !children || !counts || !nc_out ||
        !workspace || !aligned16(coords) || !aligned16(coarse_coords)) {
        set_last_error("spc_downsample_map: null or misaligned argument");
        return SPC_BAD_ARG;
    }
    if (n_batch <= 0 || n_batch > kBatchLimit || resolution <= 0 || resolution > kCoordLimit) {
        set_last_error("spc_downsample_map: n_batch %lld / resolution %d out of range",
                       (long long)n_batch, resolution);
        return SPC_BAD_ARG;
    }
    const int64_t n = nf;
    Carver c(workspace, workspace_bytes);
    int32_t* status = c.take<int32_t>(kStatusBytes / 4);
    auto* keys = c.take<unsigned long long>(n);
    auto* sk = c.take<unsigned long long>(n);
    int32_t* sv = c.take<int32_t>(n);
    int32_t* flag = c.take<int32_t>(n);
    int32_t* excl = c.take<int32_t>(n);
    int32_t* head = c.take<int32_t>(n + 1);
    int32_t* nc_dev = c.take<int32_t>(1);
    const size_t sort_bytes = radix_sort_ws_bytes(n, 8);
    char* sort_ws = c.take<char>(sort_bytes);
    const size_t scan_bytes = scan_ws_bytes(n);
    char* scan_ws = c.take<char>(scan_bytes);
    if (!c.ok) {
        set_last_error("spc_downsample_map: workspace too small");
        return SPC_OOM;
    }
    const int cbits = bits_for((resolution + 1) / 2);
    const int end_bit = 3 * cbits + bits_for(n_batch);
    const int4* c4 = reinterpret_cast<const int4*>(coords);
    SPC_HIP(fill_i32(s, status, 0, 1));
    coarse_key_kernel<<<grid_for(n, 256), 256, 0, s>>>(c4, n, n_batch, resolution, cbits, keys,
                                                       status);
    SPC_HIP(radix_sort_u64(s, keys, nullptr, sk, sv, n, end_bit, sort_ws, sort_bytes));
    head_flag_kernel<<<grid_for(n, 256), 256, 0, s>>>(sk, n, flag);
    SPC_HIP(exclusive_scan_i32(s, flag, excl, nc_dev, n, scan_ws, scan_bytes));
    downsample_assign_kernel<<<grid_for(n, 256), 256, 0, s>>>(
        sk, sv, flag, excl, n, cbits, fine_to_coarse, head, reinterpret_cast<int4*>(coarse_coords));
    downsample_children_kernel<<<grid_for(n, 256), 256, 0, s>>>(
        sv, head, nc_dev, c4, n, children, counts, stride2_taps, status);
    SPC_HIP(hipGetLastError());
    int32_t nc_host = 0;
    SPC_HIP(hipMemcpyAsync(&nc_host, nc_dev, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    const int code = read_status_word(s, status);  // synchronises
    *nc_out = nc_host;
    return code;
}

size_t spc_subdivide_workspace_bytes(int64_t n) {
    const int64_t m8 = (n > 0 ? n : 1) * 8;
    Sizer z;
    z.take<int32_t>(kStatusBytes / 4);
    z.take<int32_t>(m8);  // flags
    z.take<int32_t>(m8);  // positions
    z.take<int32_t>(1);   // total
    z.take<char>(scan_ws_bytes(m8));
    return z.used + 256;
}

int spc_subdivide_map(spc_stream_t stream, const int32_t* coords, int64_t n, const uint8_t* keep,
                      uint32_t flags, int32_t* out_coords, int32_t* parent, int64_t* m_out,
                      void* workspace, size_t workspace_bytes) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n <= 0 || n > INT32_MAX / 8) {
        set_last_error("spc_subdivide_map: n = %lld out of range", (long long)n);
        return SPC_BAD_SHAPE;
    }
    if (!coords || !out_coords || !parent || !m_out || !workspace || !aligned16(coords) ||
        !aligned16(out_coords)) {
        set_last_error("spc_subdivide_map: null or misaligned argument");
        return SPC_BAD_ARG;
    }
    const int64_t m8 = n * 8;
    Carver c(workspace, workspace_bytes);
    int32_t* status = c.take<int32_t>(kStatusBytes / 4);
    int32_t* flag = c.take<int32_t>(m8);
    int32_t* pos = c.take<int32_t>(m8);
    int32_t* total = c.take<int32_t>(1);
    const size_t scan_bytes = scan_ws_bytes(m8);
    char* scan_ws = c.take<char>(scan_bytes);
    if (!c.ok) {
        set_last_error("spc_subdivide_map: workspace too small");
        return SPC_OOM;
    }
    SPC_HIP(fill_i32(s, status, 0, 1));
    if (keep) {
        subdivide_flag_kernel<<<grid_for(m8, 256), 256, 0, s>>>(keep, m8, flag);
        SPC_HIP(exclusive_scan_i32(s, flag, pos, total, m8, scan_ws, scan_bytes));
    }
    subdivide_kernel<<<grid_for(m8, 256), 256, 0, s>>>(
        reinterpret_cast<const int4*>(coords), n, keep, pos, reinterpret_cast<int4*>(out_coords),
        parent, status);
    SPC_HIP(hipGetLastError());
    int32_t m = (int32_t)m8;
    int code = SPC_OK;
    if (keep) {
        // the survivor count comes back with the status word (one synchronisation)
        SPC_HIP(hipMemcpyAsync(&m, total, sizeof(int32_t), hipMemcpyDeviceToHost, s));
        code = read_status_word(s, status);
    } else if (flags & SPC_MAP_SYNC) {
        code = read_status_word(s, status);
    }
    *m_out = m;
    return code;
}

int spc_stride2_inverse_taps(spc_stream_t stream, const int32_t* coords,
                             const int32_t* fine_to_coarse, int64_t nf, int64_t nc,
                             int32_t* taps) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (nf < 0 || nc < 0 || nf > INT32_MAX / 8 || nc > INT32_MAX) {
        set_last_error("spc_stride2_inverse_taps: nf=%lld nc=%lld out of range", (long long)nf,
                       (long long)nc);
        return SPC_BAD_SHAPE;
    }
    if (nf == 0) return SPC_OK;
    if (!coords || !fine_to_coarse || !taps || !aligned16(coords) || !aligned16(taps)) {
        set_last_error("spc_stride2_inverse_taps: null or misaligned argument");
        return SPC_BAD_ARG;
    }
    stride2_inverse_kernel<<<grid_for(nf, 256), 256, 0, s>>>(
        reinterpret_cast<const int4*>(coords), fine_to_coarse, nf, (int32_t)nc, taps);
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_subdivide_neighbors(spc_stream_t stream, const int32_t* parent_token_major,
                            int64_t n_parent, int32_t* child_token_major) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_parent < 0 || n_parent > INT32_MAX / (8 * 27)) {
        set_last_error("spc_subdivide_neighbors: n_parent = %lld out of range", (long long)n_parent);
        return SPC_BAD_SHAPE;
    }
    if (n_parent == 0) return SPC_OK;
    if (!parent_token_major || !child_token_major) {
        set_last_error("spc_subdivide_neighbors: null table");
        return SPC_BAD_ARG;
    }
    subdivide_neighbors_kernel<<<(unsigned)ceil_div(n_parent, (int64_t)kSnParents), 256, 0, s>>>(
        parent_token_major, n_parent, child_token_major);
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_subdivide_tap_classes(spc_stream_t stream, const int32_t* parent_token_major,
                              int64_t n_parent, int64_t class_rows, int32_t* idx,
                              int32_t* row_perm) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_parent < 0 || n_parent > INT32_MAX / 64 || class_rows < n_parent || class_rows % 256 != 0 ||
        class_rows > INT32_MAX / 8) {
        set_last_error("spc_subdivide_tap_classes: n_parent=%lld class_rows=%lld (a multiple of "
                       "256, >= n_parent)", (long long)n_parent, (long long)class_rows);
        return SPC_BAD_SHAPE;
    }
    if (class_rows == 0) return SPC_OK;
    if (!parent_token_major || !idx || !row_perm) {
        set_last_error("spc_subdivide_tap_classes: null argument");
        return SPC_BAD_ARG;
    }
    const int64_t work = std::max<int64_t>(64 * n_parent, 8 * class_rows);
    subdivide_tap_classes_kernel<<<grid_for(work, 256), 256, 0, s>>>(parent_token_major, n_parent,
                                                                     class_rows, idx, row_perm);
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

int spc_compose_rows(spc_stream_t stream, const int32_t* idx, int64_t n, const int32_t* rows,
                     int64_t n_rows, int32_t* out) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (n < 0 || n_rows < 0 || n_rows > INT32_MAX) {
        set_last_error("spc_compose_rows: n=%lld n_rows=%lld out of range", (long long)n,
                       (long long)n_rows);
        return SPC_BAD_SHAPE;
    }
    if (n == 0) return SPC_OK;
    if (!idx || !out || (!rows && n_rows > 0) || !aligned16(idx) || !aligned16(out)) {
        set_last_error("spc_compose_rows: null or misaligned argument (idx / out 16-byte aligned)");
        return SPC_BAD_ARG;
    }
    const int64_t lanes = n / 4 + (n % 4);
    compose_rows_kernel<<<grid_for(lanes, 256), 256, 0, s>>>(idx, n, rows, n_rows, out);
    SPC_HIP(hipGetLastError());
    return SPC_OK;
}

}  // extern "C"
