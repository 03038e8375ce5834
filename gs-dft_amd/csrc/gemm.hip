// FP64 MFMA products. The blocked Cholesky's: C(m, n) -= sum_k A(k, m) B(k, n), with both
// operands stored k-contiguous (A(k, m) at A[m lda + k], B(k, n) at B[n ldb + k]) and C
// column-major (C(m, n) at C[n ldc + m]). That is the shape of every update of the right-looking
// factorisation of the column-major upper factor: the panel solve's block update and the trailing
// update C -= P^T P, for which only the tiles on or above the diagonal are formed (`upper`). And
// the general one of the grid density and the exchange (launch_gemm): C = alpha op(A) op(B) +
// beta C, each operand either k-contiguous or m/n-contiguous (A(m, k) at A[k lda + m], B(k, n) at
// B[k ldb + n]), batched over strided operands.
//
// Tiles of 128 x 128 per workgroup (4 waves of 64 x 64, each 4 x 4 v_mfma_f64_16x16x4f64
// accumulators), K in steps of 16 staged in LDS with two buffers: the next step's operands are
// loaded from global memory (16 consecutive k of one column per 16 lanes: 128-byte segments)
// while the current step's 64 MFMAs per wave run. The wave forms the transposed tile
// D(n, m) = sum_k B(k, n) A(k, m), so that the 16 lanes of an MFMA output row hold 16 consecutive
// m of one column of C and the read-modify-write of C goes in 128-byte segments.
#include <algorithm>

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
// gemm_cm_split: products with fewer than kSplitTiles output tiles split K into up to
// kSplitMaxSlices slices of at least kSplitMinK, for about 2 kSplitTiles workgroups.
constexpr int64_t kSplitTiles = 256, kSplitMaxSlices = 32, kSplitMinK = 256;

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

// The epilogue of every product: c <- alpha acc + beta c (c not read for beta = 0). For the
// factorisation's alpha = -1, beta = 1 that is c - acc, rounded once.
__device__ __forceinline__ void epilogue(double* c, double acc, double alpha, double beta) {
    *c = beta == 0.0 ? alpha * acc : __builtin_fma(alpha, acc, beta * *c);
}

// The step's tile of one operand through registers: kKC, stored k-contiguous (element (row, k) at
// P[row ld + k]): element e = t + 256 q is (row t / 16 + 16 q, k t % 16), so one base address and
// a uniform stride of 16 rows; otherwise row-contiguous (element (row, k) at P[k ld + row]):
// element e is (row t % 128, k t / 128 + 2 q), two 1 KB runs of 128 rows per load. Either way it
// is stored to LDS as [row][k]. kEdge guards every load (a clamped in-range address, then zeroed).
template <bool kKC, bool kEdge>
struct TileLoader {
    const double* __restrict__ P;
    int64_t ld, r0, R, K;
    double v[kLoadsPerThread];

    __device__ __forceinline__ int row_of(int q) const {
        const int t = threadIdx.x;
        return kKC ? (t >> 4) + kRowsPerLoad * q : (t & (kTile - 1));
    }
    __device__ __forceinline__ int k_of(int q) const {
        const int t = threadIdx.x;
        return kKC ? (t & 15) : (t >> 7) + 2 * q;
    }
    __device__ __forceinline__ void load(int64_t k0) {
#pragma unroll
        for (int q = 0; q < kLoadsPerThread; ++q) {
            const int64_t r = r0 + row_of(q), k = k0 + k_of(q);
            if constexpr (kEdge) {
                const int64_t rc = r < R ? r : R - 1, kc = k < K ? k : K - 1;
                const double x = kKC ? P[rc * ld + kc] : P[kc * ld + rc];
                v[q] = (r < R && k < K) ? x : 0.0;
            } else {
                v[q] = kKC ? P[r * ld + k] : P[k * ld + r];
            }
        }
    }
    __device__ __forceinline__ void store(double (*S)[kLdsK]) const {
#pragma unroll
        for (int q = 0; q < kLoadsPerThread; ++q) S[row_of(q)][k_of(q)] = v[q];
    }
};

// One 128 x 128 tile of C = alpha op(A) op(B) + beta C through registers. kEdge: the tile crosses
// the end of C or K is not a multiple of 16, so every load is guarded and the stores too.
template <bool kEdge, bool kAK = true, bool kBK = true>
__device__ __forceinline__ void gemm_tile(int64_t m0, int64_t n0, int64_t Mr, int64_t Nc,
                                          int64_t K, const double* __restrict__ A, int64_t lda,
                                          const double* __restrict__ B, int64_t ldb,
                                          double* __restrict__ C, int64_t ldc,
                                          double (*As)[kTile][kLdsK],
                                          double (*Bs)[kTile][kLdsK], double alpha,
                                          double beta) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave & 1, wn = wave >> 1;  // wave tile: m in [64 wm, +64), n in [64 wn, +64)
    const int l16 = lane & 15, l4 = lane >> 4;
    TileLoader<kAK, kEdge> la{A, lda, m0, Mr, K, {}};
    TileLoader<kBK, kEdge> lb{B, ldb, n0, Nc, K, {}};
    auto load = [&](int64_t k0) {
        la.load(k0);
        lb.load(k0);
    };
    auto store = [&](int buf) {
        la.store(As[buf]);
        lb.store(Bs[buf]);
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
                if (!kEdge || m < Mr) epilogue(col + m, acc[i][j][r], alpha, beta);
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

// The DMA path for either operand layout and any K: a k-contiguous operand's K-step tile as above
// (128 rows x 8 swizzled 16-byte chunks), a row-contiguous one's as 16 k-rows of 128 consecutive
// rows, each row-run one DMA instruction (64 lanes x 16 bytes) and padded to kRowPitch doubles so
// that the four 16-lane groups of an MFMA operand read (four k-rows) fall in different banks
// within each half-wave. The K % 16 trailing k go last, through guarded register loads into the
// same layout with zeros past K.
constexpr int kRowPitch = kTile + 16;
constexpr int kOpK = kTile * kStepK;           // doubles of a k-contiguous operand tile
constexpr int kOpR = kStepK * kRowPitch;       // doubles of a row-contiguous one
constexpr int kOpMax = kOpR > kOpK ? kOpR : kOpK;

template <bool kKC>
struct DmaOperand {
    const double* g[4];     // this lane's source for each of its four instructions, at k = 0
    int64_t kstep;          // source doubles per unit of k
    int dst[4];             // LDS doubles of each instruction's first slot
    const double* __restrict__ P;
    int64_t ld, r0, R, K;

    // Rows past R (an edge tile) read the last row instead (k-contiguous) or the last even
    // 16-byte chunk (row-contiguous: ld is even, so the chunk's second row is inside ld); they
    // feed only outputs past the end of C, which are not stored.
    __device__ __forceinline__ void init(const double* __restrict__ P_, int64_t ld_, int64_t r0_,
                                         int64_t R_, int64_t K_) {
        P = P_; ld = ld_; r0 = r0_; R = R_; K = K_;
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (kKC) {
                const int slot = (4 * q + wave) * 64 + lane, r = slot >> 3;
                const int c = (slot & 7) ^ (r & 7);
                const int64_t rg = r0 + r < R ? r0 + r : R - 1;
                g[q] = P + rg * ld + 2 * c;
                dst[q] = (4 * q + wave) * 64 * 2;
            } else {
                const int kq = wave + 4 * q;
                const int64_t last = (R - 1) & ~int64_t(1);
                const int64_t rg = r0 + 2 * lane < last ? r0 + 2 * lane : last;
                g[q] = P + kq * ld + rg;
                dst[q] = kq * kRowPitch;
            }
        }
        kstep = kKC ? 1 : ld;
    }
    __device__ __forceinline__ void dma(int64_t k0, double* __restrict__ lds) const {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            __builtin_amdgcn_global_load_lds((const void*)(g[q] + k0 * kstep),
                                             (lds_ptr)(lds + dst[q]), 16, 0, 0);
    }
    // LDS double of (row, k) of the step's tile
    __device__ __forceinline__ static int at(int row, int k) {
        if constexpr (kKC) return (8 * row + ((k >> 1) ^ (row & 7))) * 2 + (k & 1);
        else return k * kRowPitch + row;
    }
    // the trailing step [k0, K) through guarded loads, zeros past K
    __device__ __forceinline__ void tail(int64_t k0, double* __restrict__ lds) const {
        const int t = threadIdx.x;
#pragma unroll
        for (int q = 0; q < kLoadsPerThread; ++q) {
            const int row = kKC ? (t >> 4) + kRowsPerLoad * q : (t & (kTile - 1));
            const int k = kKC ? (t & 15) : (t >> 7) + 2 * q;
            const int64_t kg = k0 + k, kc = kg < K ? kg : K - 1;
            const int64_t rg = r0 + row < R ? r0 + row : R - 1;
            const double x = kKC ? P[rg * ld + kc] : P[kc * ld + rg];
            lds[at(row, k)] = kg < K ? x : 0.0;
        }
    }
};

template <bool kAK, bool kBK>
__device__ __forceinline__ void gemm_tile_dma_gen(int64_t m0, int64_t n0, int64_t Mr, int64_t Nc,
                                                  int64_t K, const double* __restrict__ A,
                                                  int64_t lda, const double* __restrict__ B,
                                                  int64_t ldb, double* __restrict__ C,
                                                  int64_t ldc, double* __restrict__ lds,
                                                  double alpha, double beta) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int l16 = lane & 15, l4 = lane >> 4;
    DmaOperand<kAK> oa;
    DmaOperand<kBK> ob;
    oa.init(A, lda, m0, Mr, K);
    ob.init(B, ldb, n0, Nc, K);
    const int64_t K0 = K - K % kStepK;
    auto bufs = [&](int buf, double** la, double** lb) {
        *la = lds + buf * 2 * kOpMax;
        *lb = *la + kOpMax;
    };

    v4d acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

    // the sub-steps [0, ksub) of one staged K step; operands of sub-step kk + 4 read during the
    // sixteen MFMAs of sub-step kk
    auto compute = [&](const double* __restrict__ la, const double* __restrict__ lb, int ksub) {
        double bn[2][4], am[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            bn[0][i] = lb[DmaOperand<kBK>::at(wn * 64 + i * 16 + l16, l4)];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            am[0][j] = la[DmaOperand<kAK>::at(wm * 64 + j * 16 + l16, l4)];
#pragma unroll
        for (int kk = 0; kk < kStepK; kk += 4) {
            if (kk >= ksub) break;
            const int cur = (kk >> 2) & 1, nxt = cur ^ 1;
            if (kk + 4 < kStepK) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    bn[nxt][i] = lb[DmaOperand<kBK>::at(wn * 64 + i * 16 + l16, kk + 4 + l4)];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    am[nxt][j] = la[DmaOperand<kAK>::at(wm * 64 + j * 16 + l16, kk + 4 + l4)];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma(bn[cur][i], am[cur][j], acc[i][j]);
        }
    };

    int buf = 0;
    if (K0 > 0) {
        double *la, *lb;
        bufs(0, &la, &lb);
        oa.dma(0, la);
        ob.dma(0, lb);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int64_t k0 = 0; k0 < K0; k0 += kStepK) {
            const bool more = k0 + kStepK < K0;
            if (more) {
                double *na, *nb;
                bufs(buf ^ 1, &na, &nb);
                oa.dma(k0 + kStepK, na);
                ob.dma(k0 + kStepK, nb);
            }
            bufs(buf, &la, &lb);
            compute(la, lb, kStepK);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            buf ^= 1;
        }
    }
    if (K0 < K) {                              // the trailing K % 16 (workgroup-uniform)
        double *la, *lb;
        bufs(buf, &la, &lb);
        oa.tail(K0, la);
        ob.tail(K0, lb);
        __syncthreads();
        compute(la, lb, (int)(K - K0));
    }
    const bool edge = m0 + kTile > Mr || n0 + kTile > Nc;       // workgroup-uniform
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t n = n0 + wn * 64 + 16 * i + l4 + 4 * r;
            if (edge && n >= Nc) continue;
            double* col = C + n * ldc;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t m = m0 + wm * 64 + 16 * j + l16;
                if (!edge || m < Mr) epilogue(col + m, acc[i][j][r], alpha, beta);
            }
        }
}

// Tile paths: kDma (interior tiles, 16-byte aligned operand rows: the DMA path), kPlain (interior
// tiles through registers), kEdge (guarded loads and stores), kDmaGen (interior tiles by DMA for
// any operand layout and any K).
enum TileMode { kDma = 0, kPlain = 1, kEdge = 2, kDmaGen = 3 };

// Strides between the operands of a batched product (blockIdx.y is the batch index) and the
// epilogue's scalars.
struct Batch {
    int64_t sa, sb, sc;
    double alpha, beta;
};

template <int kMode, bool kAK = true, bool kBK = true>
__global__ __launch_bounds__(kThreads, 2) void k_gemm_tn_sub(int64_t Mr, int64_t Nc, int64_t K,
                                                             const double* __restrict__ A,
                                                             int64_t lda,
                                                             const double* __restrict__ B,
                                                             int64_t ldb, double* __restrict__ C,
                                                             int64_t ldc, TileSet ts, Batch bt) {
    int64_t tm, tn;
    tile_of(blockIdx.x, ts, &tm, &tn);
    A += blockIdx.y * bt.sa;
    B += blockIdx.y * bt.sb;
    C += blockIdx.y * bt.sc;
    if constexpr (kMode == kDma) {
        __shared__ __align__(16) double lds[2 * 2 * kTile * kStepK];
        // the factorisation's own path: C -= A^T B
        gemm_tile_dma(tm * kTile, tn * kTile, K, A, lda, B, ldb, C, ldc, lds);
    } else if constexpr (kMode == kDmaGen) {
        __shared__ __align__(16) double lds[2 * 2 * kOpMax];
        gemm_tile_dma_gen<kAK, kBK>(tm * kTile, tn * kTile, Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                    lds, bt.alpha, bt.beta);
    } else {
        __shared__ double As[2][kTile][kLdsK];
        __shared__ double Bs[2][kTile][kLdsK];
        gemm_tile<kMode == kEdge, kAK, kBK>(tm * kTile, tn * kTile, Mr, Nc, K, A, lda, B, ldb, C,
                                            ldc, As, Bs, bt.alpha, bt.beta);
    }
}

template <int kMode, bool kAK = true, bool kBK = true>
int launch_tiles(int64_t Mr, int64_t Nc, int64_t K, const double* A, int64_t lda,
                 const double* B, int64_t ldb, double* C, int64_t ldc, TileSet ts, int64_t blocks,
                 hipStream_t s, Batch bt = Batch{0, 0, 0, -1.0, 1.0}, int64_t batch = 1) {
    if (blocks <= 0 || batch <= 0) return GSDFT_OK;
    if (blocks > INT32_MAX || batch > 65535) return fail(GSDFT_ERR_ARG, "gemm: too many tiles");
    k_gemm_tn_sub<kMode, kAK, kBK><<<dim3((unsigned)blocks, (unsigned)batch), kThreads, 0, s>>>(
        Mr, Nc, K, A, lda, B, ldb, C, ldc, ts, bt);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

// Every tile of an Mr x Nc product: the interior ones on the fast path for the layouts (DMA when
// both operands are k-contiguous with 16-byte aligned rows, else through registers), the last
// partial tile row and column guarded; K not a multiple of 16 guards them all.
template <bool kAK, bool kBK>
int launch_all_tiles(int64_t Mr, int64_t Nc, int64_t K, const double* A, int64_t lda,
                     const double* B, int64_t ldb, double* C, int64_t ldc, Batch bt,
                     int64_t batch, hipStream_t s) {
    const int64_t tiles_m = (Mr + kTile - 1) / kTile, tiles_n = (Nc + kTile - 1) / kTile;
    const int64_t fm = Mr / kTile, fn = Nc / kTile;
    const bool dma = lda % 2 == 0 && ldb % 2 == 0 && bt.sa % 2 == 0 && bt.sb % 2 == 0 &&
                     reinterpret_cast<uintptr_t>(A) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(B) % 16 == 0;
    if (dma)                                   // every tile, the edge ones included
        return launch_tiles<kDmaGen, kAK, kBK>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                               TileSet{0, 0, tiles_m, 0}, tiles_m * tiles_n, s,
                                               bt, batch);
    if (K % kStepK == 0)
        GSDFT_TRY((launch_tiles<kPlain, kAK, kBK>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                                 TileSet{0, 0, fm, 0}, fm * fn, s, bt, batch)));
    else
        GSDFT_TRY((launch_tiles<kEdge, kAK, kBK>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                                TileSet{0, 0, fm, 0}, fm * fn, s, bt, batch)));
    if (fm < tiles_m)                          // the last tile row, every column
        GSDFT_TRY((launch_tiles<kEdge, kAK, kBK>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                                TileSet{fm, 0, 1, 0}, tiles_n, s, bt, batch)));
    if (fn < tiles_n)                          // the last tile column, the full rows
        GSDFT_TRY((launch_tiles<kEdge, kAK, kBK>(Mr, Nc, K, A, lda, B, ldb, C, ldc,
                                                TileSet{0, fn, fm, 0}, fm, s, bt, batch)));
    return GSDFT_OK;
}

// C = beta C (beta = 0 writes zeros) over an Mr x Nc column-major block of each batch.
// (the grid strides over the Mr Nc elements: they can pass one grid dimension's 2^32 - 1)
__global__ void k_scale_c(int64_t Mr, int64_t Nc, double beta, double* __restrict__ C,
                          int64_t ldc, int64_t sc) {
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < Mr * Nc;
         e += (int64_t)gridDim.x * blockDim.x) {
        double* c = C + blockIdx.y * sc + (e / Mr) * ldc + e % Mr;
        *c = beta == 0.0 ? 0.0 : beta * *c;
    }
}

}  // namespace

int launch_gemm(int64_t Mr, int64_t Nc, int64_t K, double alpha, const double* A, int64_t lda,
                bool a_kc, int64_t stride_a, const double* B, int64_t ldb, bool b_kc,
                int64_t stride_b, double beta, double* C, int64_t ldc, int64_t stride_c,
                int64_t batch, hipStream_t s) {
    if (Mr <= 0 || Nc <= 0 || batch <= 0) return GSDFT_OK;
    const Batch bt{stride_a, stride_b, stride_c, alpha, beta};
    if (K <= 0) {                              // C = beta C: a product over no terms
        if (beta == 1.0) return GSDFT_OK;
        if (batch > 65535) return fail(GSDFT_ERR_ARG, "gemm: too many batches");
        const int64_t blocks = std::min<int64_t>((Mr * Nc + 255) / 256, UINT32_MAX / 256);
        k_scale_c<<<dim3((unsigned)blocks, (unsigned)batch), 256, 0, s>>>(Mr, Nc, beta, C, ldc,
                                                                         stride_c);
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    if (a_kc && b_kc) return launch_all_tiles<true, true>(Mr, Nc, K, A, lda, B, ldb, C, ldc, bt,
                                                          batch, s);
    if (a_kc) return launch_all_tiles<true, false>(Mr, Nc, K, A, lda, B, ldb, C, ldc, bt, batch,
                                                   s);
    if (b_kc) return launch_all_tiles<false, true>(Mr, Nc, K, A, lda, B, ldb, C, ldc, bt, batch,
                                                   s);
    return launch_all_tiles<false, false>(Mr, Nc, K, A, lda, B, ldb, C, ldc, bt, batch, s);
}

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

int gemm_cm(char transa, char transb, int64_t m, int64_t n, int64_t k, double alpha,
            const double* A, int64_t lda, const double* B, int64_t ldb, double beta, double* C,
            int64_t ldc, hipStream_t s) {
    return launch_gemm(m, n, k, alpha, A, lda, transa == 'T', 0, B, ldb, transb == 'N', 0, beta,
                       C, ldc, 0, 1, s);
}

namespace {

// C(i, j) = beta C(i, j) + sum over the S slices, in slice order, of part[q m n + j m + i]
// (beta = 0 does not read C).
__global__ void k_add_slices(int64_t m, int64_t n, int64_t S, const double* __restrict__ part,
                             double beta, double* __restrict__ C, int64_t ldc) {
    const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (e >= m * n) return;
    double v = 0.0;
    for (int64_t q = 0; q < S; ++q) v += part[q * m * n + e];
    double* c = C + (e / m) * ldc + e % m;
    *c = beta == 0.0 ? v : __builtin_fma(beta, *c, v);
}

}  // namespace

int64_t gemm_split_slices(int64_t m, int64_t n, int64_t k) {
    const int64_t tiles = ((m + kTile - 1) / kTile) * ((n + kTile - 1) / kTile);
    if (tiles >= kSplitTiles) return 1;
    int64_t S = (2 * kSplitTiles + tiles - 1) / tiles;
    S = S < kSplitMaxSlices ? S : kSplitMaxSlices;
    S = S < k / kSplitMinK ? S : k / kSplitMinK;
    return S < 1 ? 1 : S;
}

int gemm_cm_slices(char transa, char transb, int64_t m, int64_t n, int64_t k, double alpha,
                   const double* A, int64_t lda, const double* B, int64_t ldb, double beta,
                   double* C, int64_t ldc, int64_t S, double* part, hipStream_t s) {
    if (S <= 1 || !part || m <= 0 || n <= 0 || k < S * kStepK)
        return gemm_cm(transa, transb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, s);
    const bool a_kc = transa == 'T', b_kc = transb == 'N';
    const int64_t Ks = (k / S) / kStepK * kStepK;            // even slice offsets keep the DMA path
    const int64_t sa = a_kc ? Ks : Ks * lda, sb = b_kc ? Ks : Ks * ldb;
    GSDFT_TRY(launch_gemm(m, n, Ks, alpha, A, lda, a_kc, sa, B, ldb, b_kc, sb, 0.0, part, m, m * n,
                          S, s));
    if (k > S * Ks)                                          // the remainder, into the last slice
        GSDFT_TRY(gemm_cm(transa, transb, m, n, k - S * Ks, alpha, A + S * sa, lda, B + S * sb,
                          ldb, 1.0, part + (S - 1) * m * n, m, s));
    k_add_slices<<<(unsigned)((m * n + 255) / 256), 256, 0, s>>>(m, n, S, part, beta, C, ldc);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int gemm_cm_split(char transa, char transb, int64_t m, int64_t n, int64_t k, double alpha,
                  const double* A, int64_t lda, const double* B, int64_t ldb, double beta,
                  double* C, int64_t ldc, double* part, int64_t part_doubles, hipStream_t s) {
    int64_t S = part && m > 0 && n > 0 ? gemm_split_slices(m, n, k) : 1;
    if (S > 1 && S * m * n > part_doubles) S = part_doubles / (m * n);
    return gemm_cm_slices(transa, transb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, S, part,
                          s);
}

}  // namespace gsdft

using namespace gsdft;

extern "C" int gsdft_dgemm(int transa, int transb, int64_t m, int64_t n, int64_t k, double alpha,
                           const double* A, int64_t lda, const double* B, int64_t ldb,
                           double beta, double* C, int64_t ldc, void* stream) {
    if (m < 0 || n < 0 || k < 0 || !C || (m > 0 && n > 0 && k > 0 && (!A || !B)))
        return fail(GSDFT_ERR_ARG, "gsdft_dgemm: bad arguments");
    const bool ta = transa != 0, tb = transb != 0;
    if (ldc < (m > 1 ? m : 1) || lda < ((ta ? k : m) > 1 ? (ta ? k : m) : 1) ||
        ldb < ((tb ? n : k) > 1 ? (tb ? n : k) : 1))
        return fail(GSDFT_ERR_ARG, "gsdft_dgemm: a leading dimension is smaller than its rows");
    return gemm_cm(ta ? 'T' : 'N', tb ? 'T' : 'N', m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                   (hipStream_t)stream);
}
