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
