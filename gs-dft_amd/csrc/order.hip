// Slot order of the pairs in the three-centre passes (one lane per pair slot).
//
// Pairs are sorted by a band of I3/I2 (a factor sqrt(2) in the pair precision's smallest
// eigenvalue scale) and then by the Morton code of the product centre on a 0.5-Bohr grid (+-256
// Bohr, clamped), so that the 64 pairs of a wave are close in space and in width and the node
// screen fires for whole waves (on the 700-atom globule, a simulation of the screen puts the nodes
// evaluated at 44.8% of all with these bands, 45.9% with bands of a factor 4, 48.6% in list order;
// the per-lane floor is 40.6%). The order only decides which pairs share a wave: each pair's sums
// run over the aux records in the same sequence whatever its slot. A stable radix sort of 36-bit
// keys makes the order a pure function of the inputs.
#include <hipcub/hipcub.hpp>

#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

constexpr int kKeyBits = 36;      // 6 band bits above 30 Morton bits

__device__ __forceinline__ uint64_t spread3_10(uint32_t v) {   // 10 bits -> every third of 30
    uint64_t x = v & 0x3ff;
    x = (x | (x << 16)) & 0x30000ffull;
    x = (x | (x << 8)) & 0x300f00full;
    x = (x | (x << 4)) & 0x30c30c3ull;
    x = (x | (x << 2)) & 0x9249249ull;
    return x;
}

// rec: pair records in list order (I1 I2 I3 | Ah | P | ...), stride rec_stride doubles. With
// n_live, records from *n_live on stand for nothing: they take the largest key, so the stable
// sort puts them after every real one, in index order, and are never read.
__global__ void k_pair_keys(int64_t n, const int64_t* __restrict__ n_live,
                            const double* __restrict__ rec, int rec_stride,
                            uint64_t* __restrict__ key, int32_t* __restrict__ idx) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    idx[a] = (int32_t)a;
    if (n_live && a >= *n_live) {
        key[a] = (1ull << kKeyBits) - 1;
        return;
    }
    const double* r = rec + (int64_t)rec_stride * a;
    const double band = __builtin_fmax(__builtin_fmin(
        __builtin_floor(2.0 * log2(r[2] / r[1])) + 32.0, 63.0), 0.0);
    uint64_t code = 0;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const double c = __builtin_fmax(__builtin_fmin(__builtin_floor(2.0 * (r[9 + d] + 256.0)),
                                                       1023.0), 0.0);
        code |= spread3_10((uint32_t)c) << d;
    }
    key[a] = ((uint64_t)band << 30) | code;
}

// Group key of list entry p: min(i, j) M + max(i, j) for a live entry (the two orders of a splat
// pair, and repeats of either, share it), M^2 + p for a dead one (a group of its own). The sort
// is stable, so the entries of one key stay in list order.
__global__ void k_group_keys(int64_t n, int64_t M, const int32_t* __restrict__ pi,
                             const int32_t* __restrict__ pj, const double* __restrict__ q,
                             uint64_t* __restrict__ key, int32_t* __restrict__ idx) {
    const int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int64_t i = pi[p], j = pj[p];
    key[p] = q[p] != 0.0 ? (uint64_t)(min(i, j) * M + max(i, j)) : (uint64_t)(M * M + p);
    idx[p] = (int32_t)p;
}

// head[s] = 1 where key order position s starts a group: a new key, or, within a run of one
// key, an entry whose weight differs bitwise from the previous entry's (the entries of a group
// share one three-centre row, formed with its first entry's weight).
__global__ void k_group_heads(int64_t n, const uint64_t* __restrict__ key,
                              const int32_t* __restrict__ ent, const double* __restrict__ q,
                              int32_t* __restrict__ head) {
    const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (s >= n) return;
    bool start = s == 0 || key[s] != key[s - 1];
    if (!start)
        start = __builtin_bit_cast(uint64_t, q[ent[s]]) !=
                __builtin_bit_cast(uint64_t, q[ent[s - 1]]);
    head[s] = start ? 1 : 0;
}

// gid[s]: inclusive count of group starts up to s; ent[s]: the entry at key order position s.
__global__ void k_group_fill(int64_t n, const int32_t* __restrict__ gid,
                             const int32_t* __restrict__ head, const int32_t* __restrict__ ent,
                             int32_t* __restrict__ ent_group, int32_t* __restrict__ ent_pos,
                             int32_t* __restrict__ grp_first, int32_t* __restrict__ grp_rep,
                             int64_t* __restrict__ n_groups) {
    const int64_t s = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (s >= n) return;
    const int32_t g = gid[s] - 1, e = ent[s];
    ent_group[e] = g;
    ent_pos[e] = (int32_t)s;
    if (head[s]) {
        grp_first[g] = (int32_t)s;
        grp_rep[g] = e;
    }
    if (s == n - 1) {
        grp_first[g + 1] = (int32_t)n;
        *n_groups = g + 1;
    }
}

inline int bit_length(uint64_t v) { return v == 0 ? 1 : 64 - __builtin_clzll(v); }

}  // namespace

size_t pair_groups_scan_bytes(int64_t n) {
    size_t b = 0;
    if (hipcub::DeviceScan::InclusiveSum(nullptr, b, (const int32_t*)nullptr, (int32_t*)nullptr,
                                         (int)(n > 0 ? n : 1)) != hipSuccess)
        return 0;
    return b;
}

int launch_pair_groups(int64_t M, int64_t n, const int32_t* pi, const int32_t* pj,
                       const double* q, const PairOrderWs& po, int32_t* head, char* scan_tmp,
                       size_t scan_bytes, int32_t* ent_group, int32_t* ent_pos,
                       int32_t* grp_first, int32_t* grp_rep, int64_t* n_groups, hipStream_t s) {
    if (n > INT32_MAX) return fail(GSDFT_ERR_ARG, "pair groups: n exceeds the int32 range");
    if (n <= 0) return GSDFT_OK;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    k_group_keys<<<blocks, 256, 0, s>>>(n, M, pi, pj, q, po.key_in, po.idx_in);
    GSDFT_HIP(hipGetLastError());
    size_t b = po.sort_bytes;
    const int bits = bit_length((uint64_t)(M * M + n));
    GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(po.sort_tmp, b, po.key_in, po.key_out,
                                                 po.idx_in, po.perm, (int)n, 0, bits, s));
    k_group_heads<<<blocks, 256, 0, s>>>(n, po.key_out, po.perm, q, head);
    GSDFT_HIP(hipGetLastError());
    // the group ids go where the unsorted keys were (no longer needed)
    int32_t* gid = reinterpret_cast<int32_t*>(po.key_in);
    b = scan_bytes;
    GSDFT_HIP(hipcub::DeviceScan::InclusiveSum(scan_tmp, b, head, gid, (int)n, s));
    k_group_fill<<<blocks, 256, 0, s>>>(n, gid, head, po.perm, ent_group, ent_pos, grp_first,
                                        grp_rep, n_groups);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int pair_order_layout(Arena& ar, int64_t n, PairOrderWs* w) {
    w->key_in = ar.take<uint64_t>(n + 1);
    w->key_out = ar.take<uint64_t>(n + 1);
    w->idx_in = ar.take<int32_t>(n + 1);
    w->perm = ar.take<int32_t>(n + 1);
    w->sort_bytes = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, w->sort_bytes, (const uint64_t*)nullptr,
                                           (uint64_t*)nullptr, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)(n > 0 ? n : 1), 0,
                                           kKeyBits) !=
        hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub sort size query failed");
    w->sort_tmp = ar.take<char>(w->sort_bytes);
    return GSDFT_OK;
}

int launch_pair_order(int64_t n, const double* rec, int rec_stride, const PairOrderWs& w,
                      hipStream_t s, const int64_t* n_live) {
    if (n > INT32_MAX) return fail(GSDFT_ERR_ARG, "pair order: n exceeds the int32 range");
    if (n <= 0) return GSDFT_OK;
    k_pair_keys<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(n, n_live, rec, rec_stride, w.key_in,
                                                            w.idx_in);
    GSDFT_HIP(hipGetLastError());
    size_t b = w.sort_bytes;
    GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(w.sort_tmp, b, w.key_in, w.key_out, w.idx_in,
                                                 w.perm, (int)n, 0, kKeyBits, s));
    return GSDFT_OK;
}

}  // namespace gsdft
