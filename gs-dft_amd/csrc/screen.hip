// Chart, pair overlap, significant-pair screening and the CSR pair index.
//
// Screening follows gs_dft/screening/pairs.py: the candidate set is every ordered (i, j) (or
// j >= i in unique mode), a pair is significant when |S_ij| > eps, and the list comes out in
// ascending flat index i*M + j. Here the candidate space is cut into tiles of one row i by 256
// consecutive columns; a count pass (wave ballot + popcount) feeds a device-wide exclusive scan,
// and an emit pass recomputes S and writes each significant pair at
//   offset(tile) + (significant lanes before it in the tile),
// which is exactly its rank in flat order -- the list is ordered by construction, with no sort
// and no atomics. The overflow path collects (flat, |S|), radix-sorts by |S| descending (stable,
// so ties keep the lower flat index, as a stable argsort of -|S| does), keeps pad_to and radix-
// sorts those back by flat index.
#include <hipcub/hipcub.hpp>

#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

constexpr int kTile = 256;

__global__ void k_chart(int64_t M, const double* __restrict__ quat,
                        const double* __restrict__ log_scale, double* __restrict__ A6,
                        double* __restrict__ norm) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m >= M) return;
    Sym3 A;
    double N;
    splat_chart(quat + 4 * m, log_scale + 3 * m, &A, &N);
    double* o = A6 + 6 * m;
    o[0] = A.xx; o[1] = A.yy; o[2] = A.zz; o[3] = A.xy; o[4] = A.xz; o[5] = A.yz;
    norm[m] = N;
}

// gs_dft/screening/pairs.py:342-345 with gs_dft/coulomb/stream.py:203-215 (the centre P does not
// enter S and is not formed).
__device__ __forceinline__ double overlap(const Sym3& Ai, const Sym3& Aj, const double mui[3],
                                          const double muj[3], double Ni, double Nj) {
    const Sym3 Ah = add(Ai, Aj);
    const double d[3] = {mui[0] - muj[0], mui[1] - muj[1], mui[2] - muj[2]};
    double Ajd[3], x[3], z[3];
    matvec(Aj, d, Ajd);
    solve3(Ah, Ajd, x);
    matvec(Ai, x, z);
    const double e = d[0] * z[0] + d[1] * z[1] + d[2] * z[2];
    const double KN = Ni * Nj * exp(-e);
    return KN * kPi15 / sqrt(det3(Ah));
}

__device__ __forceinline__ void load_splat(const double* __restrict__ A6,
                                           const double* __restrict__ mu,
                                           const double* __restrict__ N, int64_t i, Sym3* A,
                                           double m[3], double* n) {
    *A = load_sym(A6 + 6 * i);
    m[0] = mu[3 * i]; m[1] = mu[3 * i + 1]; m[2] = mu[3 * i + 2];
    *n = N[i];
}

__global__ void k_overlap_list(int64_t n, const int32_t* __restrict__ pi,
                               const int32_t* __restrict__ pj, const double* __restrict__ A6,
                               const double* __restrict__ mu, const double* __restrict__ N,
                               double* __restrict__ S) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    Sym3 Ai, Aj;
    double mi[3], mj[3], ni, nj;
    load_splat(A6, mu, N, pi[a], &Ai, mi, &ni);
    load_splat(A6, mu, N, pj[a], &Aj, mj, &nj);
    S[a] = overlap(Ai, Aj, mi, mj, ni, nj);
}

struct TileGeom {
    int64_t M;
    int64_t tiles_per_row;
    int unique;
    int all;          // eps < 0: every candidate is significant, S is not evaluated
    double eps;
};

// Significance of the candidate (i, j) held by this thread; also returns |S| when evaluated.
__device__ __forceinline__ bool candidate(const TileGeom& g, int64_t i, int64_t j,
                                          const double* __restrict__ A6,
                                          const double* __restrict__ mu,
                                          const double* __restrict__ N, double* sval) {
    *sval = 0.0;
    if (j >= g.M || (g.unique && j < i)) return false;
    if (g.all) return true;
    Sym3 Ai, Aj;
    double mi[3], mj[3], ni, nj;
    load_splat(A6, mu, N, i, &Ai, mi, &ni);
    load_splat(A6, mu, N, j, &Aj, mj, &nj);
    const double s = fabs(overlap(Ai, Aj, mi, mj, ni, nj));
    *sval = s;
    return s > g.eps;
}

__global__ __launch_bounds__(kTile) void k_screen_count(TileGeom g, const double* __restrict__ A6,
                                                        const double* __restrict__ mu,
                                                        const double* __restrict__ N,
                                                        int32_t* __restrict__ counts) {
    const int64_t t = blockIdx.x;
    const int64_t i = t / g.tiles_per_row;
    const int64_t j0 = (t % g.tiles_per_row) * kTile;
    __shared__ int wave_cnt[kTile / 64];
    if (g.unique && j0 + kTile <= i) {            // whole tile below the diagonal
        if (threadIdx.x == 0) counts[t] = 0;
        return;
    }
    double s;
    const bool f = candidate(g, i, j0 + threadIdx.x, A6, mu, N, &s);
    const uint64_t mask = __ballot(f);
    if ((threadIdx.x & 63) == 0) wave_cnt[threadIdx.x >> 6] = __popcll(mask);
    __syncthreads();
    if (threadIdx.x == 0) {
        int c = 0;
        for (int w = 0; w < kTile / 64; ++w) c += wave_cnt[w];
        counts[t] = c;
    }
}

// mode 0: write (pi, pj, weight) directly; mode 1: collect (flat, |S|) for the keep-largest sort.
__global__ __launch_bounds__(kTile) void k_screen_emit(TileGeom g, const double* __restrict__ A6,
                                                       const double* __restrict__ mu,
                                                       const double* __restrict__ N,
                                                       const int64_t* __restrict__ offsets,
                                                       int mode, int64_t cap,
                                                       int32_t* __restrict__ pi,
                                                       int32_t* __restrict__ pj,
                                                       double* __restrict__ weight,
                                                       int64_t* __restrict__ flat,
                                                       double* __restrict__ val) {
    const int64_t t = blockIdx.x;
    const int64_t i = t / g.tiles_per_row;
    const int64_t j0 = (t % g.tiles_per_row) * kTile;
    if (g.unique && j0 + kTile <= i) return;
    __shared__ int wave_cnt[kTile / 64];
    const int64_t j = j0 + threadIdx.x;
    double s;
    const bool f = candidate(g, i, j, A6, mu, N, &s);
    const uint64_t mask = __ballot(f);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) wave_cnt[wave] = __popcll(mask);
    __syncthreads();
    if (!f) return;
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wave_cnt[w];
    const uint64_t lower = (lane == 0) ? 0ull : (mask & (~0ull >> (64 - lane)));
    const int64_t pos = offsets[t] + before + __popcll(lower);
    if (pos >= cap) return;
    if (mode == 0) {
        pi[pos] = (int32_t)i;
        pj[pos] = (int32_t)j;
        weight[pos] = g.unique ? (i == j ? 1.0 : 2.0) : 1.0;
    } else {
        flat[pos] = i * g.M + j;
        val[pos] = s;
    }
}

__global__ void k_fill_tail(int64_t start, int64_t end, int32_t* __restrict__ pi,
                            int32_t* __restrict__ pj, double* __restrict__ weight) {
    const int64_t a = start + blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= end) return;
    pi[a] = 0;
    pj[a] = 0;
    weight[a] = 0.0;
}

__global__ void k_decode(int64_t n, const int64_t* __restrict__ flat, int64_t M, int unique,
                         int32_t* __restrict__ pi, int32_t* __restrict__ pj,
                         double* __restrict__ weight) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int64_t f = flat[a];
    const int32_t i = (int32_t)(f / M), j = (int32_t)(f % M);
    pi[a] = i;
    pj[a] = j;
    weight[a] = unique ? (i == j ? 1.0 : 2.0) : 1.0;
}

__global__ void k_iota(int64_t n, int32_t* __restrict__ out) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a < n) out[a] = (int32_t)a;
}

// ptr[m] = first position in sorted keys[0:n) holding a key >= m, for m in [0, M].
__global__ void k_lower_bound(int64_t M, int64_t n, const int32_t* __restrict__ keys,
                              int32_t* __restrict__ ptr) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m > M) return;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (keys[mid] < m) lo = mid + 1; else hi = mid;
    }
    ptr[m] = (int32_t)lo;
}

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

int key_bits(int64_t M) {
    int b = 1;
    while ((int64_t(1) << b) < M + 1) ++b;
    return b;
}

struct ScreenWs {
    double* A6;
    double* N;
    int32_t* counts;
    int64_t* offsets;
    void* scan_tmp;
    size_t scan_bytes;
    int64_t* flat_in;
    int64_t* flat_out;
    double* val_in;
    double* val_out;
    void* sort_tmp;
    size_t sort_bytes;
};

int64_t n_tiles(int64_t M) { return M * ((M + kTile - 1) / kTile); }

bool tiles_fit(int64_t M) { return n_tiles(M) <= 2147483647LL; }

// Lays the screening workspace out over the arena (nullptr base = size query).
int layout_screen(Arena& ar, int64_t M, int64_t keep_cap, ScreenWs* w) {
    const int64_t T = n_tiles(M > 0 ? M : 1);
    w->A6 = ar.take<double>(6 * M + 1);
    w->N = ar.take<double>(M + 1);
    w->counts = ar.take<int32_t>(T);
    w->offsets = ar.take<int64_t>(T);
    w->scan_bytes = 0;
    if (hipcub::DeviceScan::ExclusiveSum(nullptr, w->scan_bytes, (const int32_t*)nullptr,
                                         (int64_t*)nullptr, (int)T) != hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub scan size query failed");
    w->scan_tmp = ar.take<char>(w->scan_bytes);
    w->flat_in = w->flat_out = nullptr;
    w->val_in = w->val_out = nullptr;
    w->sort_tmp = nullptr;
    w->sort_bytes = 0;
    if (keep_cap > 0) {
        w->flat_in = ar.take<int64_t>(keep_cap);
        w->flat_out = ar.take<int64_t>(keep_cap);
        w->val_in = ar.take<double>(keep_cap);
        w->val_out = ar.take<double>(keep_cap);
        size_t b1 = 0, b2 = 0;
        if (hipcub::DeviceRadixSort::SortPairsDescending(
                nullptr, b1, (const double*)nullptr, (double*)nullptr, (const int64_t*)nullptr,
                (int64_t*)nullptr, (int)keep_cap) != hipSuccess ||
            hipcub::DeviceRadixSort::SortKeys(nullptr, b2, (const int64_t*)nullptr,
                                              (int64_t*)nullptr, (int)keep_cap) != hipSuccess)
            return fail(GSDFT_ERR_LIB, "hipcub sort size query failed");
        w->sort_bytes = b1 > b2 ? b1 : b2;
        w->sort_tmp = ar.take<char>(w->sort_bytes);
    }
    return GSDFT_OK;
}

// Chart + count pass + scan; returns n_sig (synchronises).
int screen_scan(int64_t M, const double* quat, const double* log_scale, const double* centers,
                const TileGeom& g, ScreenWs& w, hipStream_t s, int64_t* n_sig) {
    const int64_t T = n_tiles(M);
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.N, s));
    k_screen_count<<<(unsigned)T, kTile, 0, s>>>(g, w.A6, centers, w.N, w.counts);
    GSDFT_HIP(hipGetLastError());
    size_t sb = w.scan_bytes;
    GSDFT_HIP(hipcub::DeviceScan::ExclusiveSum(w.scan_tmp, sb, w.counts, w.offsets, (int)T, s));
    int64_t last_off = 0;
    int32_t last_cnt = 0;
    GSDFT_TRY(read_back(&last_off, w.offsets + (T - 1), sizeof(int64_t), s, "screen: offsets"));
    GSDFT_TRY(read_back(&last_cnt, w.counts + (T - 1), sizeof(int32_t), s, "screen: counts"));
    *n_sig = last_off + last_cnt;
    return GSDFT_OK;
}

// ------------------------------------------------------------------ spatial candidates
// gs_dft/screening/pairs.py:167-222 builds a superset of the significant pairs from the splat
// centres (a KD-tree ball query with r_cut from grid.py:76-82) and compacts the significant ones in
// ascending flat order. Here the superset comes from a bound that holds for every splat pair:
// S_ij = p_ij exp(-e_ij) with p_ij <= 1 (det(A_i + A_j) >= 8 sqrt(det A_i det A_j)) and
// e_ij = d^T (A_i^-1 + A_j^-1)^-1 d >= |d|^2 / (1/lmin_i + 1/lmin_j), so |S_ij| > eps needs
// |d|^2 < L (1/lmin_i + 1/lmin_j), L = -ln eps. With b_i = kSpatialMargin L / lmin_i the candidate
// test is |d|^2 < b_i + b_j (the margin covers rounding). lmin_i is a lower bound of the smallest
// eigenvalue of the chart's A_i: the chart rotates by q/(|q| + 1e-12), whose rotation matrix is
// nu^2 R(u) + (1 - nu^2) I (nu the norm of the divided quaternion), so by Weyl's inequality the
// eigenvalues sit within 4 eps (1 + eps) a_max of the a_k = e^(l_k), eps = |1 - nu^2|; a splat
// whose bound is not positive is a candidate for every pair.
//
// Splats are sorted by the Morton code of their centre and cut into blocks of 64 with bounding
// boxes. One workgroup per row i: waves test whole blocks against the box (one lane per block),
// expand the live ones (one lane per member), append the candidates to an LDS list and evaluate
// S_ij on the list with every lane busy, setting bit j of the row's LDS bitmap when |S_ij| > eps.
// S_ij is the same function on the same operands (i the row) as in the dense scan, so the bitmap
// is exactly the dense scan's row; its popcount gives the row count, the exclusive scan the row
// offsets, and the emit pass writes each row's set bits in ascending j, i.e. in flat order.

constexpr double kSpatialMargin = 1.0625;
constexpr int kSpBlock = 64;              // splats per Morton block
constexpr int kSpList = 4096;             // LDS candidate list per round
constexpr int kSpExpand = kSpList / 256;  // live blocks each wave expands per round
constexpr int64_t kSpMaxM = 262144;       // bitmap row (M / 8 bytes) must fit in LDS

inline int64_t sp_words(int64_t M) { return (M + 31) / 32; }

__global__ void k_sp_prep(int64_t M, const double* __restrict__ quat,
                          const double* __restrict__ log_scale, double L,
                          double* __restrict__ b) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m >= M) return;
    const double* q = quat + 4 * m;
    const double nrm = sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    const double nu = nrm / (nrm + 1e-12);
    const double e = fabs(1.0 - nu * nu);
    const double* l = log_scale + 3 * m;
    const double amin = exp(fmin(l[0], fmin(l[1], l[2])));
    const double amax = exp(fmax(l[0], fmax(l[1], l[2])));
    const double lmin = amin - (4.0 * e * (1.0 + e) + 1e-14) * amax;
    b[m] = lmin > 0.0 ? kSpatialMargin * L / lmin : INFINITY;
}

// Bounding box of the centres (one workgroup, strided): lo (3), hi (3).
__global__ __launch_bounds__(1024) void k_sp_bbox(int64_t M, const double* __restrict__ mu,
                                                  double* __restrict__ box) {
    __shared__ double red[6][1024 / 64];
    double v[6] = {INFINITY, INFINITY, INFINITY, -INFINITY, -INFINITY, -INFINITY};
    for (int64_t m = threadIdx.x; m < M; m += blockDim.x)
        for (int c = 0; c < 3; ++c) {
            v[c] = fmin(v[c], mu[3 * m + c]);
            v[3 + c] = fmax(v[3 + c], mu[3 * m + c]);
        }
    for (int off = 32; off > 0; off >>= 1)
        for (int c = 0; c < 3; ++c) {
            v[c] = fmin(v[c], __shfl_xor(v[c], off, 64));
            v[3 + c] = fmax(v[3 + c], __shfl_xor(v[3 + c], off, 64));
        }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0)
        for (int c = 0; c < 6; ++c) red[c][wave] = v[c];
    __syncthreads();
    if (threadIdx.x < 6) {
        const int c = threadIdx.x;
        double r = red[c][0];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
            r = c < 3 ? fmin(r, red[c][w]) : fmax(r, red[c][w]);
        box[c] = r;
    }
}

__device__ __forceinline__ uint32_t spread3(uint32_t x) {      // 10 bits -> every third bit
    x &= 0x3ff;
    x = (x | (x << 16)) & 0x030000ff;
    x = (x | (x << 8)) & 0x0300f00f;
    x = (x | (x << 4)) & 0x030c30c3;
    x = (x | (x << 2)) & 0x09249249;
    return x;
}

__global__ void k_sp_morton(int64_t M, const double* __restrict__ mu,
                            const double* __restrict__ box, uint32_t* __restrict__ key,
                            int32_t* __restrict__ idx) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m >= M) return;
    uint32_t k = 0;
    for (int c = 0; c < 3; ++c) {
        const double ext = box[3 + c] - box[c];
        const double t = ext > 0.0 ? (mu[3 * m + c] - box[c]) / ext : 0.0;
        const uint32_t g = (uint32_t)fmin(fmax(t * 1024.0, 0.0), 1023.0);
        k |= spread3(g) << c;
    }
    key[m] = k;
    idx[m] = (int32_t)m;
}

// Per Morton block: members' (x, y, z, b) in sorted order, the box (lo, hi) and the largest b.
__global__ __launch_bounds__(256) void k_sp_blocks(int64_t M, const int32_t* __restrict__ perm,
                                                   const double* __restrict__ mu,
                                                   const double* __restrict__ b,
                                                   double4* __restrict__ member,
                                                   double* __restrict__ blk) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t B = m / kSpBlock;
    const bool live = m < M;
    double x = 0.0, y = 0.0, z = 0.0, bb = -INFINITY;
    if (live) {
        const int64_t j = perm[m];
        x = mu[3 * j]; y = mu[3 * j + 1]; z = mu[3 * j + 2]; bb = b[j];
        member[m] = make_double4(x, y, z, bb);
    }
    double v[7] = {live ? x : INFINITY, live ? y : INFINITY, live ? z : INFINITY,
                   live ? x : -INFINITY, live ? y : -INFINITY, live ? z : -INFINITY, bb};
    for (int off = 32; off > 0; off >>= 1)
        for (int c = 0; c < 7; ++c) {
            const double o = __shfl_xor(v[c], off, 64);
            v[c] = c < 3 ? fmin(v[c], o) : fmax(v[c], o);
        }
    if ((threadIdx.x & 63) == 0 && B * kSpBlock < M)
        for (int c = 0; c < 7; ++c) blk[8 * B + c] = v[c];
}

struct SpGeom {
    int64_t M;
    int64_t n_blocks;
    int64_t words;      // bitmap words per row
    int unique;
    double eps;
};

// One workgroup (256 lanes) per row i; dynamic LDS = the row's bitmap (words x 4 bytes).
__global__ __launch_bounds__(256) void k_sp_rows(SpGeom g, const double* __restrict__ A6,
                                                 const double* __restrict__ mu,
                                                 const double* __restrict__ Nrm,
                                                 const double* __restrict__ b,
                                                 const int32_t* __restrict__ perm,
                                                 const double4* __restrict__ member,
                                                 const double* __restrict__ blk,
                                                 uint32_t* __restrict__ bitmap,
                                                 int32_t* __restrict__ counts) {
    extern __shared__ uint32_t bits[];
    __shared__ int32_t list[kSpList];
    __shared__ int list_n;
    __shared__ int wave_cnt[4];
    const int64_t i = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t w = threadIdx.x; w < g.words; w += 256) bits[w] = 0u;
    const double mx = mu[3 * i], my = mu[3 * i + 1], mz = mu[3 * i + 2];
    const double bi = b[i];
    const Sym3 Ai = load_sym(A6 + 6 * i);
    const double mui[3] = {mx, my, mz};
    const double Ni = Nrm[i];
    int64_t next = (int64_t)wave * 64;   // next chunk of 64 blocks this wave tests
    int64_t base = 0;                     // block index of bit 0 of `pending`
    uint64_t pending = 0;                 // live blocks of the current chunk not yet expanded
    bool done = false;
    bool all_done = false;
    while (!all_done) {
        if (threadIdx.x == 0) list_n = 0;
        __syncthreads();
        for (int budget = kSpExpand; budget > 0 && !done;) {
            if (pending == 0) {
                if (next >= g.n_blocks) { done = true; break; }
                const int64_t B = next + lane;
                bool live = false;
                if (B < g.n_blocks) {
                    const double* bx = blk + 8 * B;
                    const double dx = fmax(fmax(bx[0] - mx, mx - bx[3]), 0.0);
                    const double dy = fmax(fmax(bx[1] - my, my - bx[4]), 0.0);
                    const double dz = fmax(fmax(bx[2] - mz, mz - bx[5]), 0.0);
                    live = dx * dx + dy * dy + dz * dz < (bi + bx[6]) * (1.0 + 1e-10);
                }
                pending = __ballot(live);
                base = next;
                next += 4 * 64;
                continue;
            }
            const int bit = __builtin_ctzll(pending);
            pending &= pending - 1;
            --budget;
            const int64_t m = (base + bit) * kSpBlock + lane;
            bool cand = false;
            int32_t j = 0;
            if (m < g.M) {
                j = perm[m];
                const double4 o = member[m];
                const double dx = o.x - mx, dy = o.y - my, dz = o.z - mz;
                cand = (!g.unique || j >= i) && dx * dx + dy * dy + dz * dz < bi + o.w;
            }
            const uint64_t cm = __ballot(cand);
            const int k = __popcll(cm);
            if (k == 0) continue;
            int at = 0;
            if (lane == 0) at = atomicAdd(&list_n, k);
            at = __shfl(at, 0, 64);
            const uint64_t lower = lane == 0 ? 0ull : (cm & (~0ull >> (64 - lane)));
            if (cand) list[at + __popcll(lower)] = j;
        }
        __syncthreads();
        const int n = list_n;
        for (int e = threadIdx.x; e < n; e += 256) {
            const int32_t j = list[e];
            Sym3 Aj;
            double muj[3], Nj;
            load_splat(A6, mu, Nrm, j, &Aj, muj, &Nj);
            if (fabs(overlap(Ai, Aj, mui, muj, Ni, Nj)) > g.eps)
                atomicOr(&bits[j >> 5], 1u << (j & 31));
        }
        all_done = __syncthreads_and(done ? 1 : 0) != 0;
    }
    int c = 0;
    uint32_t* row = bitmap + i * g.words;
    for (int64_t w = threadIdx.x; w < g.words; w += 256) {
        const uint32_t v = bits[w];
        row[w] = v;
        c += __popc(v);
    }
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    if (lane == 0) wave_cnt[wave] = c;
    __syncthreads();
    if (threadIdx.x == 0) counts[i] = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
}

// One wave per row: the row's set bits, in ascending j, at the row's offset.
__global__ __launch_bounds__(256) void k_sp_emit(SpGeom g, const uint32_t* __restrict__ bitmap,
                                                 const int64_t* __restrict__ offsets,
                                                 int32_t* __restrict__ pi,
                                                 int32_t* __restrict__ pj,
                                                 double* __restrict__ weight) {
    const int64_t i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= g.M) return;
    const int lane = threadIdx.x & 63;
    const uint32_t* row = bitmap + i * g.words;
    int64_t pos = offsets[i];
    for (int64_t w0 = 0; w0 < g.words; w0 += 64) {
        const int64_t w = w0 + lane;
        uint32_t v = w < g.words ? row[w] : 0u;
        const int c = __popc(v);
        int incl = c;
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        int64_t p = pos + incl - c;
        while (v) {
            const int bit = __builtin_ctz(v);
            v &= v - 1;
            const int32_t j = (int32_t)(w * 32 + bit);
            pi[p] = (int32_t)i;
            pj[p] = j;
            weight[p] = g.unique ? (i == j ? 1.0 : 2.0) : 1.0;
            ++p;
        }
        pos += __shfl(incl, 63, 64);
    }
}

struct SpatialWs {
    double* A6;
    double* N;
    double* b;
    double* box;
    uint32_t* key_in;
    uint32_t* key_out;
    int32_t* idx_in;
    int32_t* perm;
    double4* member;
    double* blk;
    uint32_t* bitmap;
    int32_t* counts;
    int64_t* offsets;
    void* tmp;
    size_t tmp_bytes;
};

int layout_spatial(Arena& ar, int64_t M, SpatialWs* w) {
    const int64_t Mx = M > 0 ? M : 1;
    const int64_t nb = (Mx + kSpBlock - 1) / kSpBlock;
    w->A6 = ar.take<double>(6 * Mx);
    w->N = ar.take<double>(Mx);
    w->b = ar.take<double>(Mx);
    w->box = ar.take<double>(8);
    w->key_in = ar.take<uint32_t>(Mx);
    w->key_out = ar.take<uint32_t>(Mx);
    w->idx_in = ar.take<int32_t>(Mx);
    w->perm = ar.take<int32_t>(Mx);
    w->member = ar.take<double4>(Mx);
    w->blk = ar.take<double>(8 * nb);
    w->bitmap = ar.take<uint32_t>(Mx * sp_words(Mx));
    w->counts = ar.take<int32_t>(Mx);
    w->offsets = ar.take<int64_t>(Mx);
    size_t b1 = 0, b2 = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, b1, (const uint32_t*)nullptr,
                                           (uint32_t*)nullptr, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)Mx) != hipSuccess ||
        hipcub::DeviceScan::ExclusiveSum(nullptr, b2, (const int32_t*)nullptr,
                                         (int64_t*)nullptr, (int)Mx) != hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub size query failed");
    w->tmp_bytes = b1 > b2 ? b1 : b2;
    w->tmp = ar.take<char>(w->tmp_bytes);
    return GSDFT_OK;
}

// Rows, bitmaps and row offsets; *n_sig = the significant count (synchronises).
int spatial_scan(int64_t M, const double* quat, const double* log_scale, const double* centers,
                 double eps, int unique, const SpatialWs& w, hipStream_t s, int64_t* n_sig) {
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.N, s));
    const double L = fmax(-log(eps), 1e-12);
    k_sp_prep<<<blocks_for(M, 256), 256, 0, s>>>(M, quat, log_scale, L, w.b);
    k_sp_bbox<<<1, 1024, 0, s>>>(M, centers, w.box);
    k_sp_morton<<<blocks_for(M, 256), 256, 0, s>>>(M, centers, w.box, w.key_in, w.idx_in);
    GSDFT_HIP(hipGetLastError());
    size_t tb = w.tmp_bytes;
    GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(w.tmp, tb, w.key_in, w.key_out, w.idx_in,
                                                 w.perm, (int)M, 0, 30, s));
    k_sp_blocks<<<blocks_for(M, 256), 256, 0, s>>>(M, w.perm, centers, w.b, w.member, w.blk);
    GSDFT_HIP(hipGetLastError());
    const SpGeom g{M, (M + kSpBlock - 1) / kSpBlock, sp_words(M), unique ? 1 : 0, eps};
    k_sp_rows<<<(unsigned)M, 256, (size_t)g.words * 4, s>>>(g, w.A6, centers, w.N, w.b, w.perm,
                                                            w.member, w.blk, w.bitmap, w.counts);
    GSDFT_HIP(hipGetLastError());
    tb = w.tmp_bytes;
    GSDFT_HIP(hipcub::DeviceScan::ExclusiveSum(w.tmp, tb, w.counts, w.offsets, (int)M, s));
    int64_t last_off = 0;
    int32_t last_cnt = 0;
    GSDFT_TRY(read_back(&last_off, w.offsets + (M - 1), sizeof(int64_t), s, "spatial: offsets"));
    GSDFT_TRY(read_back(&last_cnt, w.counts + (M - 1), sizeof(int32_t), s, "spatial: counts"));
    *n_sig = last_off + last_cnt;
    return GSDFT_OK;
}

}  // namespace

int launch_chart(int64_t M, const double* quat, const double* log_scale, double* A6, double* N,
                 hipStream_t s) {
    if (M <= 0) return GSDFT_OK;
    k_chart<<<blocks_for(M, 256), 256, 0, s>>>(M, quat, log_scale, A6, N);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace gsdft

using namespace gsdft;

extern "C" int gsdft_splat_chart(int64_t M, const double* quat, const double* log_scale,
                                 double* A6, double* norm, void* stream) {
    if (M < 0 || (M > 0 && (!quat || !log_scale || !A6 || !norm)))
        return fail(GSDFT_ERR_ARG, "gsdft_splat_chart: bad arguments");
    return launch_chart(M, quat, log_scale, A6, norm, (hipStream_t)stream);
}

extern "C" int gsdft_screen_workspace_size(int64_t M, int unique, int64_t keep_cap,
                                           size_t* bytes) {
    (void)unique;
    if (M < 0 || keep_cap < 0 || !bytes) return fail(GSDFT_ERR_ARG, "screen_workspace_size: bad arguments");
    Arena ar{nullptr, 0, 0};
    ScreenWs w;
    GSDFT_TRY(layout_screen(ar, M, keep_cap, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_overlap_pairs(int64_t M, const double* quat, const double* log_scale,
                                   const double* centers, int64_t n, const int32_t* pi,
                                   const int32_t* pj, double* S, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    if (M <= 0 || n < 0) return fail(GSDFT_ERR_ARG, "gsdft_overlap_pairs: bad sizes");
    GSDFT_TRY(check_pairs(n, "gsdft_overlap_pairs"));
    if (n == 0) return GSDFT_OK;
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    double* A6 = ar.take<double>(6 * M + 1);
    double* N = ar.take<double>(M + 1);
    if (!A6 || !N) return fail(GSDFT_ERR_WORKSPACE, "gsdft_overlap_pairs: workspace too small");
    GSDFT_TRY(launch_chart(M, quat, log_scale, A6, N, s));
    k_overlap_list<<<blocks_for(n, 256), 256, 0, s>>>(n, pi, pj, A6, centers, N, S);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

extern "C" int gsdft_screen_count(int64_t M, const double* quat, const double* log_scale,
                                  const double* centers, double eps, int unique, void* workspace,
                                  size_t workspace_bytes, int64_t* n_sig, void* stream) {
    if (M <= 0 || !n_sig || !tiles_fit(M))
        return fail(GSDFT_ERR_ARG, "gsdft_screen_count: bad arguments");
    hipStream_t s = (hipStream_t)stream;
    if (eps < 0.0) {
        *n_sig = unique ? M * (M + 1) / 2 : M * M;
        return GSDFT_OK;
    }
    Arena ar{(char*)workspace, workspace_bytes, 0};
    ScreenWs w;
    GSDFT_TRY(layout_screen(ar, M, 0, &w));
    if (!w.scan_tmp) return fail(GSDFT_ERR_WORKSPACE, "gsdft_screen_count: workspace too small");
    TileGeom g{M, (M + kTile - 1) / kTile, unique ? 1 : 0, 0, eps};
    ProfileScope prof(kProfScreen, s);
    return screen_scan(M, quat, log_scale, centers, g, w, s, n_sig);
}

extern "C" int gsdft_screen_build(int64_t M, const double* quat, const double* log_scale,
                                  const double* centers, double eps, int unique, int64_t pad_to,
                                  int32_t* pi, int32_t* pj, double* weight, void* workspace,
                                  size_t workspace_bytes, int64_t* n_sig, void* stream) {
    if (M <= 0 || pad_to < 0 || !n_sig || !tiles_fit(M) || (pad_to > 0 && (!pi || !pj || !weight)))
        return fail(GSDFT_ERR_ARG, "gsdft_screen_build: bad arguments");
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    ScreenWs w;
    GSDFT_TRY(layout_screen(ar, M, 0, &w));
    if (!w.scan_tmp) return fail(GSDFT_ERR_WORKSPACE, "gsdft_screen_build: workspace too small");
    // Every pair is significant and the pad holds them all: the list is the repeat/tile (or
    // upper-triangle) order and S is never evaluated (pairs.py:258-272). A pad below the full
    // count still needs |S| for the ranking, so it takes the evaluated path.
    const int64_t n_all = unique ? M * (M + 1) / 2 : M * M;
    const int all = (eps < 0.0 && pad_to >= n_all) ? 1 : 0;
    TileGeom g{M, (M + kTile - 1) / kTile, unique ? 1 : 0, all, eps};
    const int64_t T = n_tiles(M);
    ProfileScope prof(kProfScreen, s);
    GSDFT_TRY(screen_scan(M, quat, log_scale, centers, g, w, s, n_sig));
    const int64_t ns = *n_sig;
    if (ns <= pad_to) {
        if (ns > 0)
            k_screen_emit<<<(unsigned)T, kTile, 0, s>>>(g, w.A6, centers, w.N, w.offsets, 0,
                                                         pad_to, pi, pj, weight, nullptr, nullptr);
        if (pad_to > ns)
            k_fill_tail<<<blocks_for(pad_to - ns, 256), 256, 0, s>>>(ns, pad_to, pi, pj, weight);
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    if (ns > 2 * pad_to) {
        return fail(GSDFT_ERR_OVERFLOW,
                    "neighbor_pairs: %lld significant pairs exceed 2x the pad (%lld). Raise "
                    "screen.pad -- the run's pair list has outgrown the shape frozen at step 0.",
                    (long long)ns, (long long)(2 * pad_to));
    }
    // keep-largest: re-lay the workspace with room for every significant pair
    Arena ar2{(char*)workspace, workspace_bytes, 0};
    ScreenWs w2;
    GSDFT_TRY(layout_screen(ar2, M, ns, &w2));
    if (!w2.sort_tmp)
        return fail(GSDFT_ERR_WORKSPACE, "gsdft_screen_build: the keep-largest path needs "
                    "gsdft_screen_workspace_size(M, unique, %lld)", (long long)ns);
    // the scan results live at the same offsets in both layouts
    k_screen_emit<<<(unsigned)T, kTile, 0, s>>>(g, w.A6, centers, w.N, w.offsets, 1, ns, nullptr,
                                                 nullptr, nullptr, w2.flat_in, w2.val_in);
    GSDFT_HIP(hipGetLastError());
    size_t sb = w2.sort_bytes;
    GSDFT_HIP(hipcub::DeviceRadixSort::SortPairsDescending(w2.sort_tmp, sb, w2.val_in,
                                                           w2.val_out, w2.flat_in, w2.flat_out,
                                                           (int)ns, 0, 64, s));
    sb = w2.sort_bytes;
    GSDFT_HIP(hipcub::DeviceRadixSort::SortKeys(w2.sort_tmp, sb, w2.flat_out, w2.flat_in,
                                                (int)pad_to, 0, 64, s));
    k_decode<<<blocks_for(pad_to, 256), 256, 0, s>>>(pad_to, w2.flat_in, M, unique ? 1 : 0, pi,
                                                      pj, weight);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

extern "C" int gsdft_pair_index_workspace_size(int64_t M, int64_t n, size_t* bytes) {
    if (M < 0 || n < 0 || !bytes) return fail(GSDFT_ERR_ARG, "pair_index_workspace_size: bad arguments");
    if (n >= INT32_MAX)
        return fail(GSDFT_ERR_ARG, "pair_index_workspace_size: n exceeds the int32 range");
    GSDFT_TRY(check_pairs(n, "pair_index_workspace_size"));
    size_t sb = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, sb, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)(n > 0 ? n : 1)) != hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub sort size query failed");
    Arena ar{nullptr, 0, 0};
    ar.take<int32_t>(n + 1);
    ar.take<int32_t>(n + 1);
    ar.take<char>(sb);
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_pair_index(int64_t M, int64_t n, const int32_t* pi, const int32_t* pj,
                                int32_t* row_ptr, int32_t* row_perm, int32_t* col_ptr,
                                int32_t* col_perm, void* workspace, size_t workspace_bytes,
                                void* stream) {
    if (M <= 0 || n < 0 || !row_ptr || !col_ptr)
        return fail(GSDFT_ERR_ARG, "gsdft_pair_index: bad arguments");
    if (n >= INT32_MAX) return fail(GSDFT_ERR_ARG, "gsdft_pair_index: n exceeds the int32 range");
    GSDFT_TRY(check_pairs(n, "gsdft_pair_index"));
    hipStream_t s = (hipStream_t)stream;
    size_t sb = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, sb, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)(n > 0 ? n : 1)) != hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub sort size query failed");
    Arena ar{(char*)workspace, workspace_bytes, 0};
    int32_t* iota = ar.take<int32_t>(n + 1);
    int32_t* keys = ar.take<int32_t>(n + 1);
    void* tmp = ar.take<char>(sb);
    if (!tmp) return fail(GSDFT_ERR_WORKSPACE, "gsdft_pair_index: workspace too small");
    const int bits = key_bits(M);
    if (n > 0) {
        k_iota<<<blocks_for(n, 256), 256, 0, s>>>(n, iota);
        size_t b = sb;
        GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(tmp, b, pi, keys, iota, row_perm, (int)n, 0,
                                                     bits, s));
    }
    k_lower_bound<<<blocks_for(M + 1, 256), 256, 0, s>>>(M, n, keys, row_ptr);
    if (n > 0) {
        size_t b = sb;
        GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(tmp, b, pj, keys, iota, col_perm, (int)n, 0,
                                                     bits, s));
    }
    k_lower_bound<<<blocks_for(M + 1, 256), 256, 0, s>>>(M, n, keys, col_ptr);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

extern "C" int gsdft_screen_spatial_workspace_size(int64_t M, size_t* bytes) {
    if (M < 0 || !bytes) return fail(GSDFT_ERR_ARG, "screen_spatial_workspace_size: bad arguments");
    Arena ar{nullptr, 0, 0};
    SpatialWs w;
    GSDFT_TRY(layout_spatial(ar, M, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_screen_spatial(int64_t M, const double* quat, const double* log_scale,
                                    const double* centers, double eps, int unique, int64_t pad_to,
                                    int32_t* pi, int32_t* pj, double* weight, void* workspace,
                                    size_t workspace_bytes, int64_t* n_sig, void* stream) {
    if (M <= 0 || M > kSpMaxM || !(eps >= 0.0) || !n_sig || !quat || !log_scale || !centers ||
        (pad_to > 0 && (!pi || !pj || !weight)))
        return fail(GSDFT_ERR_ARG, "gsdft_screen_spatial: bad arguments (needs 0 < M <= %lld and "
                    "eps >= 0)", (long long)kSpMaxM);
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    SpatialWs w;
    GSDFT_TRY(layout_spatial(ar, M, &w));
    if (!w.tmp) return fail(GSDFT_ERR_WORKSPACE, "gsdft_screen_spatial: workspace too small");
    ProfileScope prof(kProfScreen, s);
    GSDFT_TRY(spatial_scan(M, quat, log_scale, centers, eps, unique, w, s, n_sig));
    if (pad_to < 0) return GSDFT_OK;
    const int64_t ns = *n_sig;
    if (ns > pad_to)
        return fail(GSDFT_ERR_FALLBACK, "gsdft_screen_spatial: %lld significant pairs exceed the "
                    "pad (%lld); the keep-largest list comes from gsdft_screen_build",
                    (long long)ns, (long long)pad_to);
    const SpGeom g{M, (M + kSpBlock - 1) / kSpBlock, sp_words(M), unique ? 1 : 0, eps};
    if (ns > 0)
        k_sp_emit<<<(unsigned)((M + 3) / 4), 256, 0, s>>>(g, w.bitmap, w.offsets, pi, pj, weight);
    if (pad_to > ns)
        k_fill_tail<<<blocks_for(pad_to - ns, 256), 256, 0, s>>>(ns, pad_to, pi, pj, weight);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}
