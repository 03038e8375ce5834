// FP64 MFMA product of the blocked Cholesky: C(m, n) -= sum_k A(k, m) B(k, n), with both operands
// stored k-contiguous (A(k, m) at A[m lda + k], B(k, n) at B[n ldb + k]) and C column-major
// (C(m, n) at C[n ldc + m]). That is the shape of every update of the right-looking factorisation
// of the column-major upper factor: the panel solve's block update and the trailing update
// C -= P^T P, for which only the tiles on or above the diagonal are formed (`upper`).
//
// Tiles of 128 x 128 per workgroup (4 waves of 64 x 64, each 4 x 4 v_mfma_f64_16x16x4f64
// accumulators), K in steps of 16 staged in LDS with two buffers: the next step's operands are
// loaded from global memory (16 consecutive k of one column per 16 lanes: 128-byte segments)
// while the current step's 64 MFMAs per wave run. The wave forms the transposed tile
// D(n, m) = sum_k B(k, n) A(k, m), so that the 16 lanes of an MFMA output row hold 16 consecutive
// m of one column of C and the read-modify-write of C goes in 128-byte segments.
#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

typedef double v4d __attribute__((ext_vector_type(4)));

// D (16 x 16) += A (16 x 4) B (4 x 16): lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]
// and holds D[l / 16 + 4 r][l % 16] in register r.
__device__ __forceinline__ v4d mfma(double a, double b, v4d c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

constexpr int kTile = 128;
constexpr int kThreads = 256;                 // 4 waves: 2 (m) x 2 (n) of 64 x 64
constexpr int kStepK = 16;
constexpr int kLdsK = kStepK + 1;             // padded rows: the 16 operand rows of a read differ in bank
constexpr int kLoadsPerThread = kTile * kStepK / kThreads;
constexpr int kRowsPerLoad = kThreads / kStepK;

// Which tiles a launch covers: every tile of a tm_count-row grid (column-major over block ids,
// starting at tile (tm0, tn0)), or (upper) the tiles with tm <= tn of a tm_count-square grid.
struct TileSet {
    int64_t tm0, tn0;
    int64_t tm_count;
    int upper;
};

// The tiles with tm <= tn of a T-square grid, in bands of kBand tile columns: band c (columns
// [kBand c, kBand c + w), w = kBand but the last) lists its full rows tm < kBand c row by row, then
// its triangle. Workgroups dispatched together then cover a few rows of one band and share both
// operand panels (in L2 and the MALL) instead of walking a whole column of A panels.
constexpr int64_t kBand = 16;

__host__ __device__ inline void upper_tile_of(int64_t b, int64_t T, int64_t* tm, int64_t* tn) {
    // full bands before band c hold sum_{c' < c} (kBand^2 c' + kBand (kBand + 1) / 2) tiles
    const double a = 0.5 * kBand * kBand, bq = 0.5 * kBand * (kBand + 1) - a;
    int64_t c = (int64_t)((-bq + sqrt(bq * bq + 4.0 * a * (double)b)) / (2.0 * a));
    auto before = [&](int64_t cc) { return (kBand * kBand * cc * (cc - 1)) / 2
                                           + cc * (kBand * (kBand + 1) / 2); };
    const int64_t bands = (T + kBand - 1) / kBand;
    if (c > bands - 1) c = bands - 1;
    while (c > 0 && before(c) > b) --c;
    while (c + 1 < bands && before(c + 1) <= b) ++c;
    const int64_t w = T - kBand * c < kBand ? T - kBand * c : kBand;
    int64_t r = b - before(c);
    const int64_t full = kBand * c * w;
    if (r < full) {
        *tm = r / w;
        *tn = kBand * c + r % w;
        return;
    }
    r -= full;
    int64_t u = 0;
    while (r >= w - u) {                    // triangle row u holds w - u tiles
        r -= w - u;
        ++u;
    }
    *tm = kBand * c + u;
    *tn = kBand * c + u + r;
}

__device__ __forceinline__ void tile_of(int64_t b, const TileSet& ts, int64_t* tm, int64_t* tn) {
    if (!ts.upper) {
        *tm = ts.tm0 + b % ts.tm_count;
        *tn = ts.tn0 + b / ts.tm_count;
        return;
    }
    upper_tile_of(b, ts.tm_count, tm, tn);
    *tm += ts.tm0;
    *tn += ts.tn0;
}

// One 128 x 128 tile of C. kEdge: the tile crosses the end of C or K is not a multiple of 16, so
// every load is guarded (a clamped in-range address, then zeroed); interior tiles load straight.
template <bool kEdge>
__device__ __forceinline__ void gemm_tile(int64_t m0, int64_t n0, int64_t Mr, int64_t Nc,
                                          int64_t K, const double* __restrict__ A, int64_t lda,
                                          const double* __restrict__ B, int64_t ldb,
                                          double* __restrict__ C, int64_t ldc,
                                          double (*As)[kTile][kLdsK],
                                          double (*Bs)[kTile][kLdsK]) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave & 1, wn = wave >> 1;  // wave tile: m in [64 wm, +64), n in [64 wn, +64)
    const int l16 = lane & 15, l4 = lane >> 4;
    // global -> registers: element e = t + 256 q is (row t / 16 + 16 q, k t % 16) of the step's
    // tile, so one base address per operand and a uniform stride of 16 rows
    double ra[kLoadsPerThread], rb[kLoadsPerThread];
    const int row0 = t >> 4, kk0 = t & 15;
    const double* __restrict__ pa = A + (m0 + row0) * lda + kk0;
    const double* __restrict__ pb = B + (n0 + row0) * ldb + kk0;
    const int64_t sa = kRowsPerLoad * lda, sb = kRowsPerLoad * ldb;
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int q = 0; q < kLoadsPerThread; ++q) {
            if constexpr (kEdge) {
                const int64_t k = k0 + kk0;
                const int64_t m = m0 + row0 + kRowsPerLoad * q, n = n0 + row0 + kRowsPerLoad * q;
                const int64_t kc = k < K ? k : K - 1;
                const double va = A[(m < Mr ? m : Mr - 1) * lda + kc];
                const double vb = B[(n < Nc ? n : Nc - 1) * ldb + kc];
                ra[q] = (m < Mr && k < K) ? va : 0.0;
                rb[q] = (n < Nc && k < K) ? vb : 0.0;
            } else {
                ra[q] = pa[q * sa + k0];
                rb[q] = pb[q * sb + k0];
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < kLoadsPerThread; ++q) {
            As[buf][row0 + kRowsPerLoad * q][kk0] = ra[q];
            Bs[buf][row0 + kRowsPerLoad * q][kk0] = rb[q];
        }
    };

    v4d acc[4][4];                            // [n sub-tile][m sub-tile]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int64_t k0 = 0; k0 < K; k0 += kStepK) {
        const bool more = k0 + kStepK < K;
        if (more) load(k0 + kStepK);
#pragma unroll
        for (int kk = 0; kk < kStepK; kk += 4) {
            double bn[4], am[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) bn[i] = Bs[buf][wn * 64 + i * 16 + l16][kk + l4];
#pragma unroll
            for (int j = 0; j < 4; ++j) am[j] = As[buf][wm * 64 + j * 16 + l16][kk + l4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma(bn[i], am[j], acc[i][j]);
        }
        if (more) store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // acc[i][j][r] = D(n, m) with n = n0 + 64 wn + 16 i + l4 + 4 r, m = m0 + 64 wm + 16 j + l16
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + wn * 64 + 16 * i + l4 + 4 * r;
            if (kEdge && n >= Nc) continue;
            double* col = C + n * ldc;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t m = m0 + wm * 64 + 16 * j + l16;
                if (!kEdge || m < Mr) col[m] -= acc[i][j][r];
            }
        }
}

// Interior tiles with the operands moved global -> LDS by global_load_lds_dwordx4 (no staging
// registers, no wait before an LDS store): each operand's K-step tile is 128 rows x 8 chunks of 16
// bytes (two consecutive k), chunk c of row r stored at slot 8 r + (c ^ (r & 7)) so that the 16
// rows an MFMA operand read touches fall in different banks. One DMA instruction fills 64
// consecutive slots (lane l the slot base + l: 8 rows, their 8 chunks permuted), 4 per thread and
// operand per K-step.
typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ void gemm_tile_dma(int64_t m0, int64_t n0, int64_t K,
                                              const double* __restrict__ A, int64_t lda,
                                              const double* __restrict__ B, int64_t ldb,
                                              double* __restrict__ C, int64_t ldc,
                                              double* __restrict__ lds) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int l16 = lane & 15, l4 = lane >> 4;
    constexpr int kOp = kTile * kStepK;       // doubles per operand tile
    // DMA q of this wave fills slots [(4 q + wave) 64, +64): row r = slot / 8, physical chunk
    // slot % 8 holds logical chunk (slot % 8) ^ (r & 7)
    const double* ga[4];
    const double* gb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int slot = (4 * q + wave) * 64 + lane, r = slot >> 3, c = (slot & 7) ^ (r & 7);
        ga[q] = A + (m0 + r) * lda + 2 * c;
        gb[q] = B + (n0 + r) * ldb + 2 * c;
    }
    auto dma = [&](int64_t k0, int buf) {
        double* la = lds + buf * 2 * kOp;
        double* lb = la + kOp;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int base = (4 * q + wave) * 64 * 2;          // doubles
            __builtin_amdgcn_global_load_lds((const void*)(ga[q] + k0), (lds_ptr)(la + base), 16,
                                             0, 0);
            __builtin_amdgcn_global_load_lds((const void*)(gb[q] + k0), (lds_ptr)(lb + base), 16,
                                             0, 0);
        }
    };
    // LDS double of (row, k): slot 8 row + ((k >> 1) ^ (row & 7)), then k & 1
    auto at = [](int row, int k) { return (8 * row + ((k >> 1) ^ (row & 7))) * 2 + (k & 1); };

    v4d acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

    dma(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int buf = 0;
    for (int64_t k0 = 0; k0 < K; k0 += kStepK) {
        const bool more = k0 + kStepK < K;
        if (more) dma(k0 + kStepK, buf ^ 1);
        const double* la = lds + buf * 2 * kOp;
        const double* lb = la + kOp;
        // operands of sub-step kk + 4 are read while the 16 MFMAs of sub-step kk run
        double bn[2][4], am[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) bn[0][i] = lb[at(wn * 64 + i * 16 + l16, l4)];
#pragma unroll
        for (int j = 0; j < 4; ++j) am[0][j] = la[at(wm * 64 + j * 16 + l16, l4)];
#pragma unroll
        for (int kk = 0; kk < kStepK; kk += 4) {
            const int cur = (kk >> 2) & 1, nxt = cur ^ 1;
            if (kk + 4 < kStepK) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    bn[nxt][i] = lb[at(wn * 64 + i * 16 + l16, kk + 4 + l4)];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    am[nxt][j] = la[at(wm * 64 + j * 16 + l16, kk + 4 + l4)];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma(bn[cur][i], am[cur][j], acc[i][j]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        buf ^= 1;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + wn * 64 + 16 * i + l4 + 4 * r;
            double* col = C + n * ldc;
#pragma unroll
            for (int j = 0; j < 4; ++j) col[m0 + wm * 64 + 16 * j + l16] -= acc[i][j][r];
        }
}

// Tile paths: kDma (interior tiles, 16-byte aligned operand rows: the DMA path), kPlain (interior
// tiles through registers), kEdge (guarded loads and stores).
enum TileMode { kDma = 0, kPlain = 1, kEdge = 2 };

template <int kMode>
__global__ __launch_bounds__(kThreads, 2) void k_gemm_tn_sub(int64_t Mr, int64_t Nc, int64_t K,
                                                             const double* __restrict__ A,
                                                             int64_t lda,
                                                             const double* __restrict__ B,
                                                             int64_t ldb, double* __restrict__ C,
                                                             int64_t ldc, TileSet ts) {
    int64_t tm, tn;
    tile_of(blockIdx.x, ts, &tm, &tn);
    if constexpr (kMode == kDma) {
        __shared__ __align__(16) double lds[2 * 2 * kTile * kStepK];
        gemm_tile_dma(tm * kTile, tn * kTile, K, A, lda, B, ldb, C, ldc, lds);
    } else {
        __shared__ double As[2][kTile][kLdsK];
        __shared__ double Bs[2][kTile][kLdsK];
        gemm_tile<kMode == kEdge>(tm * kTile, tn * kTile, Mr, Nc, K, A, lda, B, ldb, C, ldc, As,
                                  Bs);
    }
}

template <int kMode>
int launch_tiles(int64_t Mr, int64_t Nc, int64_t K, const double* A, int64_t lda,
                 const double* B, int64_t ldb, double* C, int64_t ldc, TileSet ts, int64_t blocks,
                 hipStream_t s) {
    if (blocks <= 0) return GSDFT_OK;
    if (blocks > INT32_MAX) return fail(GSDFT_ERR_ARG, "gemm_tn_sub: too many tiles");
    k_gemm_tn_sub<kMode><<<(unsigned)blocks, kThreads, 0, s>>>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                                              ts);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace

int launch_gemm_tn_sub(int64_t Mr, int64_t Nc, int64_t K, const double* A, int64_t lda,
                       const double* B, int64_t ldb, double* C, int64_t ldc, bool upper,
                       hipStream_t s) {
    if (Mr <= 0 || Nc <= 0 || K <= 0) return GSDFT_OK;
    const int64_t tiles_m = (Mr + kTile - 1) / kTile, tiles_n = (Nc + kTile - 1) / kTile;
    if (upper && tiles_m != tiles_n)
        return fail(GSDFT_ERR_ARG, "gemm_tn_sub: the upper-tile product needs a square C");
    if (K % kStepK != 0) {                     // every tile takes the guarded path
        const TileSet all{0, 0, tiles_m, upper ? 1 : 0};
        return launch_tiles<kEdge>(Mr, Nc, K, A, lda, B, ldb, C, ldc, all,
                                   upper ? tiles_n * (tiles_n + 1) / 2 : tiles_m * tiles_n, s);
    }
    // interior tiles (inside C) unguarded -- by DMA when every operand row starts 16-byte
    // aligned -- and the last partial tile row and column guarded
    const bool dma = lda % 2 == 0 && ldb % 2 == 0 && reinterpret_cast<uintptr_t>(A) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(B) % 16 == 0;
    auto interior = [&](TileSet ts, int64_t blocks) {
        return dma ? launch_tiles<kDma>(Mr, Nc, K, A, lda, B, ldb, C, ldc, ts, blocks, s)
                   : launch_tiles<kPlain>(Mr, Nc, K, A, lda, B, ldb, C, ldc, ts, blocks, s);
    };
    const int64_t fm = Mr / kTile, fn = Nc / kTile;
    if (upper) {
        GSDFT_TRY(interior(TileSet{0, 0, fn, 1}, fn * (fn + 1) / 2));
        if (fn < tiles_n)                      // the last tile column, rows 0 .. its diagonal
            GSDFT_TRY(launch_tiles<kEdge>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                          TileSet{0, fn, tiles_n, 0}, tiles_n, s));
        return GSDFT_OK;
    }
    GSDFT_TRY(interior(TileSet{0, 0, fm, 0}, fm * fn));
    if (fm < tiles_m)                          // the last tile row, every column
        GSDFT_TRY(launch_tiles<kEdge>(Mr, Nc, K, A, lda, B, ldb, C, ldc, TileSet{fm, 0, 1, 0},
                                      tiles_n, s));
    if (fn < tiles_n)                          // the last tile column, the full rows
        GSDFT_TRY(launch_tiles<kEdge>(Mr, Nc, K, A, lda, B, ldb, C, ldc, TileSet{0, fn, fm, 0},
                                      fm, s));
    return GSDFT_OK;
}

}  // namespace gsdft
