// Screened exact exchange through density fitting (RI-K), gs_dft/coulomb/ri.py:497-544:
//   D[P,o,o'] = sum over listed pairs a = (i, k) of w_a C_io C_ko' (P|a),
//   E_K = -Tr((V + lam I)^-1 M),   M_PQ = sum_oo' D[P,o,o'] D[Q,o,o'].
// With the Cholesky factor L L^T = V + lam I this is E_K = -||L^-1 D||_F^2 over the k^2 columns
// (o, o'). An orthogonal change of the column basis keeps the norm, so the columns are stored as
// the symmetric part, (D_oo' + D_o'o)/sqrt2 for o < o' and D_oo on the diagonal (k(k+1)/2
// columns), followed by the antisymmetric part (D_oo' - D_o'o)/sqrt2 for o < o'. On a symmetric
// pair list (every live (i, k, w) has its (k, i, w)) each D_P is symmetric up to round-off and the
// antisymmetric columns are dropped.
//
// The list's entries are grouped by unordered splat pair {i, k} and weight: (i, k) and (k, i)
// share one product Gaussian, so the three-centre passes run once per group (on a symmetric list
// half the entries), the block's row of a group serves all its entries, and the reverse takes the
// sum of their cotangents.
// Forward, per chunk of W aux functions (centre-grouped slot order):
//   Bt (groups x W)     the screened three-centre block (k_exch_block_pairs, dfj.hip)
//   Y[i][l][o']         = sum over pairs a of row i of Bt[g_a][l] C[k_a][o']   (k_exch_spmm, FP64
//                         MFMA over the row's block columns and gathered C rows)
//   D_P = C^T Y_P       one FP64 GEMM per chunk: k x (W k) x M
//   Dt[:, P]            packed columns of D_P                                    (k_exch_pack)
// then Wt = Dt L^-T (blocked substitution over the packed-column right-hand sides,
// trsm_right_upper) and E_K = -sum Wt^2.
// Reverse with seed dE_K = 1: Dbar_t = -2 Wt L^-1 (trsm), then per chunk Dbar_P (k_exch_unpack),
// with the forward's Y (and Y') kept in the workspace when they fit, else recomputed,
//   dC    += Y_P Dbar_P^T + Y'_P Dbar_P      Y'[m][l][o] = sum over pairs a of column m of
//                                            Bt[a][l] C[i_a][o] (= Y on a symmetric list)
//   Ybar_P = C Dbar_P,   Tbar[a][l] = Ybar[i_a][l] . C[k_a]            (k_exch_sddmm, FP64 MFMA)
//   and the three-centre reverse with the per-(P, group) cotangent, the sum of its entries' Tbar
//   (dfj.hip), for the splat gradients. On a symmetric list Dbar_P is symmetric, so the entries
//   of a group share Tbar = (C Dbar_P C^T)[i][k]: the sampled product runs once per group (over
//   the groups as a CSR by lower splat) and the reverse takes that row times the entry count.
//   Every sum runs in a fixed order (no atomics); the dense products and the triangular solves
//   are the library's own FP64 MFMA kernels (gemm.hip, trsm_right_upper).
#include <algorithm>

#include <cmath>

#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

inline unsigned nblk(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

// x <- alpha x over n doubles.
__global__ void k_scale(int64_t n, double alpha, double* __restrict__ x) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) x[i] *= alpha;
}

constexpr double kRsqrt2 = 0.70710678118654752440;
constexpr int kRedBlocks = 1024;
constexpr double kChunkBytes = 8.0 * 1024 * 1024 * 1024;   // per-chunk buffers of the default chunk
constexpr double kStoreBytes = 32.0 * 1024 * 1024 * 1024;   // Y (and Y') kept for the reverse
constexpr int64_t kSplitMax = 32;                           // K slices of the dC GEMM

// FP64 MFMA v_mfma_f64_16x16x4f64, D (16 x 16) += A (16 x 4) B (4 x 16), one wave: lane l supplies
// A[l % 16][l / 16] and B[l / 16][l % 16] and holds D[l / 16 + 4 r][l % 16] in its register r
// (checked with a one-wave probe of known operands on MI355X).
typedef double v4d __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4d mfma16x16x4(double a, double b, v4d c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

constexpr int kColPad = 16;     // entries of the per-position partner arrays past n (splat 0)
constexpr int kMfAux = 32;      // aux per wave (two 16-row tiles)
constexpr int kMfOrb = 96;      // orbitals per wave in the Y product (six 16-column tiles)
constexpr int kMfK = 96;        // orbitals held in registers per pass of the Tbar product
inline int64_t padded_cols(int64_t k) { return (k + 15) / 16 * 16; }

// Y[i][l][o] = sum_{r in [ptr[i], ptr[i+1])} Bt[perm[r] * ldb + l] C[col[r] * k + o] for l < W,
// o < k (perm[r] = the block row of CSR position r, its pair group; col[r] = its partner splat),
// with C read from Cp, its rows padded to kp = 16 ceil(k / 16) columns (zeros). Per row i this is
// the product of the row's block columns (W x deg) and its gathered C rows (deg x kp): grid
// (rows, ceil(W / (4 kMfAux)), column blocks), 4 waves, each wave a 32 x 16 NT tile of Y_i in
// 2 NT MFMA accumulators (NT = 6 for the full 96-column blocks, the remainder in one more
// launch), K = 4 pairs per MFMA. The row's pairs go through LDS in stages of kSpPairs: the
// workgroup loads a stage's 128 block columns and 16 NT-wide C rows once (wave w the pairs
// w, w + 4, ...) into one of two buffers while the MFMAs run on the other.
constexpr int kSpPairs = 8;       // 33 KB of LDS: three workgroups per CU (16: two, 2.5% slower)
constexpr int kSpAux = 4 * kMfAux;              // aux columns per workgroup
// Padded LDS rows: each row starts 128 bytes (mod 256) after the previous one, so the two rows an
// MFMA operand read takes per half-wave fall in different banks.
constexpr int kSpLdA = kSpAux + 16;
__host__ __device__ constexpr int sp_ld_c(int nt) { return 16 * nt + (nt % 2 == 0 ? 16 : 0); }

template <int NT>
__global__ __launch_bounds__(256) void k_exch_spmm(int64_t W, int64_t k, int64_t kp, int64_t ldb,
                                                   int64_t obase,
                                                   const int32_t* __restrict__ ptr,
                                                   const int32_t* __restrict__ perm,
                                                   const int32_t* __restrict__ col,
                                                   const double* __restrict__ Bt,
                                                   const double* __restrict__ Cp,
                                                   double* __restrict__ Y) {
    constexpr int kLdC = sp_ld_c(NT);
    __shared__ double As[2][kSpPairs][kSpLdA];
    __shared__ double Cs[2][kSpPairs][kLdC];
    const int64_t i = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kq = lane >> 4, c16 = lane & 15;
    const int64_t lbase = (int64_t)blockIdx.y * kSpAux;
    const int64_t ob = obase + (int64_t)blockIdx.z * (16 * NT);
    v4d acc[2][NT];
#pragma unroll
    for (int ta = 0; ta < 2; ++ta)
#pragma unroll
        for (int to = 0; to < NT; ++to) acc[ta][to] = v4d{0.0, 0.0, 0.0, 0.0};
    const int64_t r0 = ptr[i], r1 = ptr[i + 1];
    // Stage at CSR position rs: wave w loads pairs w + 4 j (j < kSpPairs / 4) into registers. The
    // pairs' indices come one stage earlier from one vector load (lane j: perm, lane kPw + j: col;
    // vector rather than scalar loads, whose counter the LDS reads of the MFMAs share) and are
    // broadcast with readlane. Every load reads an in-range address (positions past the row
    // clamped to its last one, columns past W to W - 1, C columns past the block to its last);
    // the values that stand for nothing are zeroed when the stage is written to LDS, so the
    // loads stay in flight through the current stage's MFMAs.
    constexpr int kPw = kSpPairs / 4;                           // pairs per wave and stage
    double sa[kPw][2], sc[kPw][2];
    int64_t staged = 0;                                         // position of the loaded stage
    const int64_t la0 = min(lbase + lane, W - 1), la1 = min(lbase + 64 + lane, W - 1);
    const bool in0 = lbase + lane < W, in1 = lbase + 64 + lane < W;
    const int oc0 = min(lane, 16 * NT - 1), oc1 = min(64 + lane, 16 * NT - 1);
    int idx = 0;                                                // indices of the next stage
    auto load_idx = [&](int64_t rs) {
        const int64_t r = rs + wave + 4 * (lane % kPw);
        const int64_t rc = r < r1 ? r : r1 - 1;
        if (lane < 2 * kPw) idx = lane < kPw ? perm[rc] : col[rc];
    };
    auto load = [&](int64_t rs) {
        staged = rs;
#pragma unroll
        for (int j = 0; j < kPw; ++j) {
            const int64_t a = __builtin_amdgcn_readlane(idx, j);
            const int64_t c = __builtin_amdgcn_readlane(idx, kPw + j);
            const double* __restrict__ ba = Bt + a * ldb;
            const double* __restrict__ cb = Cp + c * kp + ob;
            sa[j][0] = ba[la0];
            sa[j][1] = ba[la1];
            sc[j][0] = cb[oc0];
            sc[j][1] = cb[oc1];
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < kPw; ++j) {
            const int p = wave + 4 * j;
            const bool has = staged + p < r1;
            As[buf][p][lane] = has && in0 ? sa[j][0] : 0.0;
            As[buf][p][64 + lane] = has && in1 ? sa[j][1] : 0.0;
            if (lane < 16 * NT) Cs[buf][p][lane] = sc[j][0];
            if (64 + lane < 16 * NT) Cs[buf][p][64 + lane] = sc[j][1];
        }
    };
    if (r0 < r1) {
        load_idx(r0);
        load(r0);
        load_idx(r0 + kSpPairs);
        store(0);
    }
    __syncthreads();
    int buf = 0;
    for (int64_t rs = r0; rs < r1; rs += kSpPairs) {          // workgroup-uniform
        const bool more = rs + kSpPairs < r1;
        if (more) {
            load(rs + kSpPairs);
            load_idx(rs + 2 * kSpPairs);
        }
#pragma unroll
        for (int k4 = 0; k4 < kSpPairs / 4; ++k4) {
            const int p = 4 * k4 + kq;
            const double a0 = As[buf][p][wave * kMfAux + c16];
            const double a1 = As[buf][p][wave * kMfAux + 16 + c16];
            double bc[NT];
#pragma unroll
            for (int to = 0; to < NT; ++to) bc[to] = Cs[buf][p][to * 16 + c16];
#pragma unroll
            for (int to = 0; to < NT; ++to) {
                acc[0][to] = mfma16x16x4(a0, bc[to], acc[0][to]);
                acc[1][to] = mfma16x16x4(a1, bc[to], acc[1][to]);
            }
        }
        if (more) store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    const int64_t lw = lbase + (int64_t)wave * kMfAux;
    const int64_t Wk = W * k;
#pragma unroll
    for (int ta = 0; ta < 2; ++ta)
#pragma unroll
        for (int to = 0; to < NT; ++to) {
            const int64_t o = ob + to * 16 + c16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t l = lw + ta * 16 + kq + 4 * r;
                if (l < W && o < k) Y[i * Wk + l * k + o] = acc[ta][to][r];
            }
        }
}

// Cp[m][j] = C[m][j] for j < k, 0 for k <= j < kp.
__global__ void k_pad_cols(int64_t M, int64_t k, int64_t kp, const double* __restrict__ C,
                           double* __restrict__ Cp) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= M * kp) return;
    const int64_t m = t / kp, j = t - m * kp;
    Cp[t] = j < k ? C[m * k + j] : 0.0;
}

// col[r] = partner[perm[r]]: the partner splat of every CSR position, and splat 0 in the
// kColPad padding entries after position n (read, never used, by the last pair tile).
__global__ void k_csr_partner(int64_t n, const int32_t* __restrict__ perm,
                              const int32_t* __restrict__ partner, int32_t* __restrict__ col) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r < n) col[r] = partner[perm[r]];
    else if (r < n + kColPad) col[r] = 0;
}

// The leading dimension of the packed columns: K2 rounded up to even, so that every column starts
// 16-byte aligned (the triangular solves stage them by DMA); the padding row stays zero.
inline int64_t packed_ld(int64_t K2) { return K2 + (K2 & 1); }

// The leading dimension of the per-chunk D_P blocks: k rounded up to even (16-byte aligned
// columns for the DMA path of the products that read them).
__host__ __device__ inline int64_t dblock_ld(int64_t k) { return k + (k & 1); }

// Packed columns of D_P (P the aux of slot q0 + l): Dfull[o + kd (l k + o')] = D_P[o][o'];
// Dt[j + ldd P] with j = o'(o'+1)/2 + o for the symmetric part (o <= o') and
// k(k+1)/2 + o'(o'-1)/2 + o for the antisymmetric part (o < o', only when !sym).
__global__ void k_exch_pack(int64_t W, int64_t k, int64_t ldd, int sym, int64_t q0, int64_t N,
                            int64_t G, const double* __restrict__ Dfull, double* __restrict__ Dt) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t kk = k * k;
    if (t >= W * kk) return;
    const int64_t l = t / kk, rem = t - l * kk;
    const int64_t op = rem / k, o = rem - op * k;
    if (o > op) return;
    const int64_t P = aux_of_slot(q0 + l, N, G);
    const int64_t kd = dblock_ld(k);
    const double* Dl = Dfull + l * k * kd;
    double* col = Dt + ldd * P;
    const double d1 = Dl[o + kd * op], d2 = Dl[op + kd * o];
    const int64_t js = op * (op + 1) / 2 + o;
    if (o == op) {
        col[js] = d1;
    } else {
        col[js] = (d1 + d2) * kRsqrt2;
        if (!sym) col[k * (k + 1) / 2 + op * (op - 1) / 2 + o] = (d1 - d2) * kRsqrt2;
    }
}

// Reverse of k_exch_pack: Dbar[o + kd (l k + o')] = dE/dD_P[o][o'] and, for a non-null E, its
// block transpose E[o' + kd (l k + o)].
__global__ void k_exch_unpack(int64_t W, int64_t k, int64_t ldd, int sym, int64_t q0, int64_t N,
                              int64_t G, const double* __restrict__ Dbt, double* __restrict__ Dbar,
                              double* __restrict__ E) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t kk = k * k;
    if (t >= W * kk) return;
    const int64_t l = t / kk, rem = t - l * kk;
    const int64_t op = rem / k, o = rem - op * k;
    const int64_t P = aux_of_slot(q0 + l, N, G);
    const double* col = Dbt + ldd * P;
    const int64_t lo = o < op ? o : op, hi = o < op ? op : o;
    double v = col[hi * (hi + 1) / 2 + lo];
    if (o != op) {
        v *= kRsqrt2;
        if (!sym) {
            const double a = col[k * (k + 1) / 2 + hi * (hi - 1) / 2 + lo] * kRsqrt2;
            v += (o < op) ? a : -a;
        }
    }
    const int64_t kd = dblock_ld(k);
    Dbar[o + kd * (l * k + op)] = v;
    if (E) E[op + kd * (l * k + o)] = v;
}

// Tbar[inv[a] * ldt + l] = sum_o Ybar[i][l][o] C[k_a][o] for the pairs a of row i and l < W
// (k_a = col[r] for the CSR position r of a; C read from the padded Cp). Per row i this is the
// product Ybar_i (W x kp) Cg^T (kp x deg) sampled at the row's pairs: grid (rows,
// ceil(W / (4 kMfAux))), 4 waves, each wave 32 aux x 16 pairs per MFMA pair tile, K = 4 orbitals
// per step. Per pass of 4 NS orbitals (NS = kMfK / 4 for the full passes, the remainder in one
// more launch) the wave holds its Ybar block in registers and walks the row's pair tiles; a pass
// after the first adds to Tbar (same lane, passes in order), so every sum has a fixed order. The
// tiles' C rows go through LDS (loaded once per workgroup, wave w the pairs w + 4 j, into one of
// two buffers while the MFMAs run on the other); the next tile's column indices and output rows
// are loaded one tile ahead.
constexpr int kSdPairs = 16;
// Padded LDS rows: row p starts 32 bytes (mod 256) after row p - 1, so the 16 rows of four
// consecutive orbitals an MFMA operand read takes fill the banks twice over without conflicts.
__host__ __device__ constexpr int sd_ld_c(int ns) { return 4 * ns + (36 - (4 * ns) % 32) % 32; }

template <int NS>
__global__ __launch_bounds__(256, 3) void k_exch_sddmm(int64_t W, int64_t k, int64_t kp,
                                                     int64_t ldt, int64_t oc_begin,
                                                     int64_t oc_end, int first,
                                                     const int32_t* __restrict__ ptr,
                                                     const int32_t* __restrict__ perm,
                                                     const int32_t* __restrict__ col,
                                                     const int32_t* __restrict__ inv,
                                                     const double* __restrict__ Ybar,
                                                     const double* __restrict__ Cp,
                                                     double* __restrict__ Tbar) {
    constexpr int kW = 4 * NS;                  // orbitals per pass
    constexpr int kLd = sd_ld_c(NS);
    __shared__ double Cs[2][kSdPairs][kLd];
    const int64_t i = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kq = lane >> 4, c16 = lane & 15;
    const int64_t lw = (int64_t)blockIdx.y * (4 * kMfAux) + (int64_t)wave * kMfAux;
    const int64_t Wk = W * k;
    const int64_t r0 = ptr[i], r1 = ptr[i + 1];
    if (r0 >= r1) return;                       // workgroup-uniform: an empty row writes nothing
    auto clampr = [&](int64_t r) { return r < r1 ? r : r1 - 1; };
    // every C load reads an in-range address (positions past the row clamped to its last one,
    // orbitals past the pass to its last); the products of pairs past the row are never stored
    const int o0 = min(lane, kW - 1), o1 = min(64 + lane, kW - 1);
    for (int64_t oc = oc_begin; oc < oc_end; oc += kW) {
        const bool store = first && oc == oc_begin;
        double ya[2][NS];
#pragma unroll
        for (int ta = 0; ta < 2; ++ta) {
            const int64_t l = lw + ta * 16 + c16;
#pragma unroll
            for (int s4 = 0; s4 < NS; ++s4) {
                const int64_t o = oc + 4 * s4 + kq;
                ya[ta][s4] = (l < W && o < k) ? Ybar[i * Wk + l * k + o] : 0.0;
            }
        }
        int idx = 0;                            // lanes j < 4: col of pair wave + 4 j of a tile
        double sc[4][2];
        auto load_idx = [&](int64_t rb) {
            if (lane < 4) idx = col[clampr(rb + wave + 4 * lane)];
        };
        auto load_c = [&]() {                  // the tile whose columns idx holds
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t c = __builtin_amdgcn_readlane(idx, j);
                const double* __restrict__ cb = Cp + c * kp + oc;
                sc[j][0] = cb[o0];
                sc[j][1] = cb[o1];
            }
        };
        auto store_c = [&](int buf) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int p = wave + 4 * j;
                if (lane < kW) Cs[buf][p][lane] = sc[j][0];
                if (64 + lane < kW) Cs[buf][p][64 + lane] = sc[j][1];
            }
        };
        load_idx(r0);
        load_c();
        load_idx(r0 + kSdPairs);
        int64_t orow = inv[perm[clampr(r0 + c16)]];    // Tbar row of this lane's pair
        int32_t pnext = perm[clampr(r0 + kSdPairs + c16)];      // its pair in the next tile
        store_c(0);
        __syncthreads();
        int buf = 0;
        for (int64_t rb = r0; rb < r1; rb += kSdPairs) {       // workgroup-uniform
            // the next tiles' loads run unconditionally (clamped, so past the last tile they read
            // the row's last pair and go unused): no branch splits the loop body, and every index
            // a load needs arrived an iteration earlier
            load_c();
            load_idx(rb + 2 * kSdPairs);
            const int32_t pn2 = perm[clampr(rb + 2 * kSdPairs + c16)];
            v4d acc[2] = {v4d{0.0, 0.0, 0.0, 0.0}, v4d{0.0, 0.0, 0.0, 0.0}};
#pragma unroll
            for (int s4 = 0; s4 < NS; ++s4) {
                const double bv = Cs[buf][c16][4 * s4 + kq];
                acc[0] = mfma16x16x4(ya[0][s4], bv, acc[0]);
                acc[1] = mfma16x16x4(ya[1][s4], bv, acc[1]);
            }
            const int64_t orow_next = inv[pnext];
            if (rb + c16 < r1) {
                double* __restrict__ out = Tbar + orow * ldt;
#pragma unroll
                for (int ta = 0; ta < 2; ++ta)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t l = lw + ta * 16 + kq + 4 * r;
                        if (l < W) out[l] = store ? acc[ta][r] : out[l] + acc[ta][r];
                    }
            }
            store_c(buf ^ 1);
            __syncthreads();
            buf ^= 1;
            orow = orow_next;
            pnext = pn2;
        }
    }
}

// part[b] = sum of x[i]^2 over block b's contiguous range (fixed order per block).
__global__ __launch_bounds__(256) void k_sumsq_part(int64_t count, const double* __restrict__ x,
                                                    double* __restrict__ part) {
    __shared__ double red[256];
    const int64_t per = (count + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = blockIdx.x * per;
    const int64_t b1 = std::min<int64_t>(count, b0 + per);
    double s = 0.0;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) s = __builtin_fma(x[i], x[i], s);
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(1024) void k_sum_scaled(int64_t m, const double* __restrict__ part,
                                                     double scale, double* __restrict__ out) {
    __shared__ double red[1024];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < m; i += 1024) s += part[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = scale * red[0];
}

// out[e] += sum over s < S of part[s * count + e], in order of s.
__global__ void k_sum_slices(int64_t count, int64_t S, const double* __restrict__ part,
                             double* __restrict__ out) {
    const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (e >= count) return;
    double v = out[e];
    for (int64_t q = 0; q < S; ++q) v += part[q * count + e];
    out[e] = v;
}

// out[r] = src[idx[r]].
__global__ void k_gather_i32(int64_t n, const int32_t* __restrict__ idx,
                             const int32_t* __restrict__ src, int32_t* __restrict__ out) {
    const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (r < n) out[r] = src[idx[r]];
}

// A symmetric list's pair groups as a CSR by lower splat, for its sampled cotangents: the groups
// (key order) run by lower splat, then upper splat, the dead ones (q = 0) last. gcol[g] = the
// upper splat of live group g (zero past them and in the kColPad entries past n), giota[g] = g.
__global__ void k_group_cols(int64_t n, const int64_t* __restrict__ n_groups,
                             const int32_t* __restrict__ rep, const int32_t* __restrict__ pi,
                             const int32_t* __restrict__ pj, const double* __restrict__ q,
                             int32_t* __restrict__ gcol, int32_t* __restrict__ giota) {
    const int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (g >= n + kColPad) return;
    int32_t c = 0;
    if (g < *n_groups) {
        const int32_t e = rep[g];
        if (q[e] != 0.0) c = max(pi[e], pj[e]);
    }
    gcol[g] = c;
    if (g < n) giota[g] = (int32_t)g;
}

// gptr[i], i <= M: the number of live groups whose lower splat is below i (a binary search over the
// groups in key order, a dead group counting as row M).
__global__ void k_group_ptr(int64_t M, const int64_t* __restrict__ n_groups,
                            const int32_t* __restrict__ rep, const int32_t* __restrict__ pi,
                            const int32_t* __restrict__ pj, const double* __restrict__ q,
                            int32_t* __restrict__ gptr) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i > M) return;
    int64_t lo = 0, hi = *n_groups;
    while (lo < hi) {
        const int64_t mid = (lo + hi) / 2;
        const int32_t e = rep[mid];
        const int64_t row = q[e] != 0.0 ? min(pi[e], pj[e]) : M;
        if (row < i)
            lo = mid + 1;
        else
            hi = mid;
    }
    gptr[i] = (int32_t)lo;
}

__global__ void k_fill0(int64_t n, double* __restrict__ out) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) out[i] = 0.0;
}

// Aux functions per chunk: the caller's choice, else as many as keep the chunk's buffers that
// grow with it (block, Y / Y', D_P blocks) near kChunkBytes, a multiple of 64. (The reverse
// moments are bounded by the pair count alone.)
int64_t exch_chunk(int64_t M, int64_t k, int64_t N, int64_t n, bool sym, bool grads,
                   int64_t req) {
    if (req > 0) return std::min(req, N);
    const double ys = (grads && !sym) ? 2.0 : 1.0;
    const double per = 8.0 * ((double)n + ys * (double)M * (double)k + ys * (double)k * (double)k);
    int64_t Pc = (int64_t)(kChunkBytes / per);
    Pc = (Pc / 64) * 64;
    if (Pc < 64) Pc = 64;
    return std::min(Pc, N);
}

// With gradients, the forward keeps Y (and Y' on a non-symmetric list) for every chunk when they
// fit in kStoreBytes, so the reverse needs neither the block nor the pair-sparse products again.
bool exch_store(int64_t M, int64_t k, int64_t N, bool sym, bool grads, bool recompute) {
    return grads && !recompute &&
           8.0 * (double)M * (double)N * (double)k * (sym ? 1.0 : 2.0) <= kStoreBytes;
}

// K slices of the dC GEMM (its k x M output is a handful of tiles; the K = W k dimension is long):
// enough for ~512 tiles in flight, at most kSplitMax and one slice per aux function.
int64_t dc_slices(int64_t k, int64_t M, int64_t W) {
    const int64_t tiles = ((k + 127) / 128) * ((M + 127) / 128);
    int64_t S = (512 + tiles - 1) / tiles;
    S = std::min<int64_t>(std::min<int64_t>(S, kSplitMax), W);
    return S < 1 ? 1 : S;
}

struct ExchWs {
    ExchTcWs tc;
    double *Dt, *Bt, *Y, *Yp, *Ys, *Yps, *Dfull, *Ebar, *part, *red;
    int32_t *row_col, *col_row;       // partner splat per CSR position (rows: pj, columns: pi)
    int32_t *row_grp, *col_grp;       // pair group (block row) per CSR position
    int32_t *gptr, *gcol, *giota;     // symmetric list: the groups as a CSR by lower splat
    double* Cp;                       // C with rows padded to padded_cols(k) columns
};

int layout_exchange(Arena& ar, int64_t M, int64_t k, int64_t N, int64_t n, bool sym, bool grads,
                    bool recompute, int64_t Pc, ExchWs* w) {
    GSDFT_TRY(exch_tc_layout(ar, M, N, n, Pc, grads, &w->tc));
    const int64_t K2 = sym ? k * (k + 1) / 2 : k * k;
    GSDFT_TRY(check_items(packed_ld(K2) * N, "exchange", "the packed columns (K2 x N_aux)"));
    GSDFT_TRY(check_items(M * padded_cols(k), "exchange", "the padded orbitals (M x k)"));
    GSDFT_TRY(check_items(Pc * k * k, "exchange", "an aux chunk's D blocks (W x k x k)"));
    const bool store = exch_store(M, k, N, sym, grads, recompute);
    w->Dt = ar.take<double>(packed_ld(K2) * N + 1);
    w->Bt = ar.take<double>(n * Pc + 1);
    w->Y = ar.take<double>(M * Pc * k + 1);
    w->Yp = (grads && !sym && !store) ? ar.take<double>(M * Pc * k + 1) : nullptr;
    w->Ys = store ? ar.take<double>(M * N * k + 1) : nullptr;
    w->Yps = (store && !sym) ? ar.take<double>(M * N * k + 1) : nullptr;
    w->Dfull = ar.take<double>(dblock_ld(k) * k * Pc + 1);
    w->Ebar = (grads && !sym) ? ar.take<double>(dblock_ld(k) * k * Pc + 1) : nullptr;
    w->part = grads ? ar.take<double>(kSplitMax * k * M + 1) : nullptr;
    w->red = ar.take<double>(kRedBlocks);
    w->Cp = ar.take<double>(M * padded_cols(k) + 1);
    w->row_col = ar.take<int32_t>(n + kColPad);
    w->col_row = sym ? nullptr : ar.take<int32_t>(n + kColPad);
    w->row_grp = ar.take<int32_t>(n + 1);
    w->col_grp = sym ? nullptr : ar.take<int32_t>(n + 1);
    const bool gcsr = sym && grads;
    w->gptr = gcsr ? ar.take<int32_t>(M + 2) : nullptr;
    w->gcol = gcsr ? ar.take<int32_t>(n + kColPad) : nullptr;
    w->giota = gcsr ? ar.take<int32_t>(n + 1) : nullptr;
    return GSDFT_OK;
}

// dC^T (k x M, column-major = row-major dC) += alpha Dbar (k x W k, leading dimension
// dblock_ld(k)) Y^T-view (W k x M, ld W k), as S K-slices of Ws = W / S aux functions (the
// remainder joins the last slice) into part, then summed in slice order.
int dc_gemm(int64_t k, int64_t M, int64_t W, double alpha, const double* Dbar, const double* Y,
            double* part, double* dC, hipStream_t s) {
    const int64_t S = dc_slices(k, M, W), Ws = W / S, Wk = W * k, kd = dblock_ld(k);
    GSDFT_TRY(launch_gemm(k, M, Ws * k, alpha, Dbar, kd, false, kd * Ws * k, Y, Wk, true, Ws * k,
                          0.0, part, k, k * M, S, s));
    const int64_t rem = W - S * Ws;
    if (rem > 0)
        GSDFT_TRY(gemm_cm('N', 'N', k, M, rem * k, alpha, Dbar + kd * (S * Ws * k), kd,
                          Y + S * Ws * k, Wk, 1.0, part + (S - 1) * k * M, k, s));
    k_sum_slices<<<nblk(k * M, 256), 256, 0, s>>>(k * M, S, part, dC);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int launch_spmm(int64_t M, int64_t W, int64_t k, int64_t ldb, const int32_t* ptr,
                const int32_t* perm, const int32_t* col, const double* Bt, const double* Cp,
                double* Y, hipStream_t s) {
    const int64_t kp = padded_cols(k);
    const int64_t full = kp / kMfOrb, tail = (kp % kMfOrb) / 16;
    profile_begin(kProfExchSparse, s);
    if (full > 0) {
        dim3 grid((unsigned)M, nblk(W, 4 * kMfAux), (unsigned)full);
        k_exch_spmm<kMfOrb / 16><<<grid, 256, 0, s>>>(W, k, kp, ldb, 0, ptr, perm, col, Bt, Cp,
                                                      Y);
    }
    if (tail > 0) {
        dim3 grid((unsigned)M, nblk(W, 4 * kMfAux), 1);
        const int64_t ob = full * kMfOrb;
        // the remainder pass: 16 * tail orbitals
        switch (tail) {
        case 1:
            k_exch_spmm<1><<<grid, 256, 0, s>>>(W, k, kp, ldb, ob, ptr, perm, col, Bt, Cp, Y);
            break;
        case 2:
            k_exch_spmm<2><<<grid, 256, 0, s>>>(W, k, kp, ldb, ob, ptr, perm, col, Bt, Cp, Y);
            break;
        case 3:
            k_exch_spmm<3><<<grid, 256, 0, s>>>(W, k, kp, ldb, ob, ptr, perm, col, Bt, Cp, Y);
            break;
        case 4:
            k_exch_spmm<4><<<grid, 256, 0, s>>>(W, k, kp, ldb, ob, ptr, perm, col, Bt, Cp, Y);
            break;
        default:
            k_exch_spmm<5><<<grid, 256, 0, s>>>(W, k, kp, ldb, ob, ptr, perm, col, Bt, Cp, Y);
            break;
        }
    }
    profile_end(kProfExchSparse, s);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int launch_sddmm(int64_t M, int64_t W, int64_t k, int64_t ldt, const int32_t* ptr,
                 const int32_t* perm, const int32_t* col, const int32_t* inv,
                 const double* Ybar, const double* Cp, double* Tbar, hipStream_t s) {
    const int64_t kp = padded_cols(k);
    const int64_t full = kp / kMfK * kMfK, tail = (kp - full) / 4;     // tail: K steps, 4 .. 20
    dim3 grid((unsigned)M, nblk(W, 4 * kMfAux));
    profile_begin(kProfExchSparse, s);
    if (full > 0)
        k_exch_sddmm<kMfK / 4><<<grid, 256, 0, s>>>(W, k, kp, ldt, 0, full, 1, ptr, perm, col, inv,
                                                   Ybar, Cp, Tbar);
    if (tail > 0) {
        const int first = full == 0 ? 1 : 0;
#define GSDFT_SDDMM_TAIL(NS)                                                                    \
    k_exch_sddmm<NS><<<grid, 256, 0, s>>>(W, k, kp, ldt, full, kp, first, ptr, perm, col, inv, \
                                          Ybar, Cp, Tbar)
        switch (tail) {
        case 4: GSDFT_SDDMM_TAIL(4); break;
        case 8: GSDFT_SDDMM_TAIL(8); break;
        case 12: GSDFT_SDDMM_TAIL(12); break;
        case 16: GSDFT_SDDMM_TAIL(16); break;
        default: GSDFT_SDDMM_TAIL(20); break;
        }
#undef GSDFT_SDDMM_TAIL
    }
    profile_end(kProfExchSparse, s);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace

}  // namespace gsdft

using namespace gsdft;

extern "C" int gsdft_exchange_workspace_size(int64_t M, int64_t k, int64_t N, int64_t n,
                                             int symmetric, int grads, int64_t aux_chunk,
                                             int recompute, size_t* bytes) {
    if (M <= 0 || k <= 0 || N <= 0 || n < 0 || aux_chunk < 0 || !bytes)
        return fail(GSDFT_ERR_ARG, "exchange_workspace_size: bad arguments");
    GSDFT_TRY(check_pairs(n, "exchange_workspace_size"));
    const bool sym = symmetric != 0, gr = grads != 0;
    const int64_t Pc = exch_chunk(M, k, N, n, sym, gr, aux_chunk);
    Arena ar{nullptr, 0, 0};
    ExchWs w;
    GSDFT_TRY(layout_exchange(ar, M, k, N, n, sym, gr, recompute != 0, Pc, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_exchange(int64_t M, const double* quat, const double* log_scale,
                              const double* centers, int64_t k, const double* C, int64_t N,
                              const double* log_alpha, const double* aux_centers,
                              const double* chol, int64_t n, const int32_t* pi, const int32_t* pj,
                              const double* weight, const int32_t* row_ptr,
                              const int32_t* row_perm, const int32_t* col_ptr,
                              const int32_t* col_perm, int symmetric, int64_t aux_chunk,
                              int recompute, double omega, double* energy, double* dquat,
                              double* dlog_scale, double* dcenters, double* dC, void* workspace,
                              size_t workspace_bytes, void* stream) {
    const bool grads = dquat != nullptr;
    if (M <= 0 || k <= 0 || N <= 0 || n < 0 || aux_chunk < 0 || !quat || !log_scale ||
        !centers || !C || !log_alpha || !aux_centers || !chol || !energy || !row_ptr ||
        (n > 0 && (!pi || !pj || !row_perm)) ||
        (grads && (!dlog_scale || !dcenters || !dC || !col_ptr || (n > 0 && !col_perm))))
        return fail(GSDFT_ERR_ARG, "gsdft_exchange: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_exchange"));
    if (!(omega >= 0.0) || std::isinf(omega))
        return fail(GSDFT_ERR_ARG, "gsdft_exchange: omega must be finite and >= 0");
    hipStream_t s = (hipStream_t)stream;
    const bool sym = symmetric != 0;
    const int64_t Pc = exch_chunk(M, k, N, n, sym, grads, aux_chunk);
    Arena ar{(char*)workspace, workspace_bytes, 0};
    ExchWs w;
    GSDFT_TRY(layout_exchange(ar, M, k, N, n, sym, grads, recompute != 0, Pc, &w));
    if (!w.red) return fail(GSDFT_ERR_WORKSPACE, "gsdft_exchange: workspace too small");
    w.tc.table = omega > 0.0 ? long_range_table(omega) : coulomb_table();
    GSDFT_TRY(exch_tc_prologue(M, quat, log_scale, centers, N, log_alpha, aux_centers, n, pi, pj,
                               weight, grads, w.tc, s));
    if (n == 0) {                       // D = 0: E_K = 0 and every gradient vanishes
        k_fill0<<<1, 1, 0, s>>>(1, energy);
        GSDFT_HIP(hipGetLastError());
        if (grads) {
            k_fill0<<<nblk(M * k, 256), 256, 0, s>>>(M * k, dC);
            GSDFT_HIP(hipGetLastError());
            GSDFT_TRY(exch_tc_finish(M, 0, pi, pj, weight, quat, log_scale, centers, row_ptr,
                                     row_perm, col_ptr, col_perm, dquat, dlog_scale, dcenters,
                                     w.tc, s));
        }
        return GSDFT_OK;
    }
    k_csr_partner<<<nblk(n + kColPad, 256), 256, 0, s>>>(n, row_perm, pj, w.row_col);
    k_gather_i32<<<nblk(n, 256), 256, 0, s>>>(n, row_perm, w.tc.ent_group, w.row_grp);
    k_pad_cols<<<nblk(M * padded_cols(k), 256), 256, 0, s>>>(M, k, padded_cols(k), C, w.Cp);
    GSDFT_HIP(hipGetLastError());
    if (!sym) {
        k_csr_partner<<<nblk(n + kColPad, 256), 256, 0, s>>>(n, col_perm, pi, w.col_row);
        k_gather_i32<<<nblk(n, 256), 256, 0, s>>>(n, col_perm, w.tc.ent_group, w.col_grp);
        GSDFT_HIP(hipGetLastError());
    } else if (grads) {
        k_group_cols<<<nblk(n + kColPad, 256), 256, 0, s>>>(n, w.tc.n_groups_dev, w.tc.grp_rep,
                                                            pi, pj, w.tc.q, w.gcol, w.giota);
        k_group_ptr<<<nblk(M + 1, 256), 256, 0, s>>>(M, w.tc.n_groups_dev, w.tc.grp_rep, pi, pj,
                                                     w.tc.q, w.gptr);
        GSDFT_HIP(hipGetLastError());
    }
    const int64_t G = (N % M == 0) ? N / M : 1;
    const int64_t K2 = sym ? k * (k + 1) / 2 : k * k, ldd = packed_ld(K2);
    const bool store = exch_store(M, k, N, sym, grads, recompute != 0);
    k_fill0<<<nblk(ldd * N, 256), 256, 0, s>>>(ldd * N, w.Dt);
    GSDFT_HIP(hipGetLastError());
    for (int64_t q0 = 0; q0 < N; q0 += Pc) {
        const int64_t W = std::min(Pc, N - q0);
        double* Yc = store ? w.Ys + M * q0 * k : w.Y;
        GSDFT_TRY(exch_tc_block(M, N, q0, W, aux_centers, n, Pc, w.Bt, w.tc, s));
        GSDFT_TRY(launch_spmm(M, W, k, Pc, row_ptr, w.row_grp, w.row_col, w.Bt, w.Cp, Yc, s));
        if (store && !sym)
            GSDFT_TRY(launch_spmm(M, W, k, Pc, col_ptr, w.col_grp, w.col_row, w.Bt, w.Cp,
                                  w.Yps + M * q0 * k, s));
        profile_begin(kProfExchGemm, s);
        GSDFT_TRY(gemm_cm('N', 'T', k, W * k, M, 1.0, w.Cp, padded_cols(k), Yc, W * k, 0.0,
                          w.Dfull, dblock_ld(k), s));
        profile_end(kProfExchGemm, s);
        k_exch_pack<<<nblk(W * k * k, 256), 256, 0, s>>>(W, k, ldd, sym ? 1 : 0, q0, N, G, w.Dfull,
                                                         w.Dt);
        GSDFT_HIP(hipGetLastError());
    }
    // Wt = Dt L^-T: chol is the row-major lower factor, i.e. the column-major upper L^T.
    profile_begin(kProfExchTrsm, s);
    // (the block buffer is idle until the reverse pass: it holds the solve's K-slices)
    GSDFT_TRY(trsm_right_upper(s, false, N, chol, N, w.Dt, K2, ldd, w.Bt, n * Pc));
    profile_end(kProfExchTrsm, s);
    k_sumsq_part<<<kRedBlocks, 256, 0, s>>>(ldd * N, w.Dt, w.red);
    GSDFT_HIP(hipGetLastError());
    k_sum_scaled<<<1, 1024, 0, s>>>(kRedBlocks, w.red, -1.0, energy);
    GSDFT_HIP(hipGetLastError());
    if (!grads) return GSDFT_OK;

    // Dbar_t = -2 Wt L^-1
    profile_begin(kProfExchTrsm, s);
    // (the scaling by -2 is exact, so it may come before the solve)
    k_scale<<<nblk(ldd * N, 256), 256, 0, s>>>(ldd * N, -2.0, w.Dt);
    GSDFT_HIP(hipGetLastError());
    GSDFT_TRY(trsm_right_upper(s, true, N, chol, N, w.Dt, K2, ldd, w.Bt, n * Pc));
    profile_end(kProfExchTrsm, s);
    k_fill0<<<nblk(M * k, 256), 256, 0, s>>>(M * k, dC);
    GSDFT_HIP(hipGetLastError());
    for (int64_t q0 = 0; q0 < N; q0 += Pc) {
        const int64_t W = std::min(Pc, N - q0);
        k_exch_unpack<<<nblk(W * k * k, 256), 256, 0, s>>>(W, k, ldd, sym ? 1 : 0, q0, N, G, w.Dt,
                                                           w.Dfull, w.Ebar);
        GSDFT_HIP(hipGetLastError());
        const double* Yc = w.Y;
        const double* Ypc = w.Yp;
        if (store) {
            Yc = w.Ys + M * q0 * k;
            Ypc = sym ? nullptr : w.Yps + M * q0 * k;
        } else {
            GSDFT_TRY(exch_tc_block(M, N, q0, W, aux_centers, n, Pc, w.Bt, w.tc, s));
            GSDFT_TRY(launch_spmm(M, W, k, Pc, row_ptr, w.row_grp, w.row_col, w.Bt, w.Cp, w.Y,
                                  s));
            if (!sym)
                GSDFT_TRY(launch_spmm(M, W, k, Pc, col_ptr, w.col_grp, w.col_row, w.Bt, w.Cp,
                                      w.Yp, s));
        }
        profile_begin(kProfExchGemm, s);
        // dC += Y_P Dbar_P^T (+ Y'_P Dbar_P; the same term again on a symmetric list)
        GSDFT_TRY(dc_gemm(k, M, W, sym ? 2.0 : 1.0, w.Dfull, Yc, w.part, dC, s));
        if (!sym) GSDFT_TRY(dc_gemm(k, M, W, 1.0, w.Ebar, Ypc, w.part, dC, s));
        // Ybar (Wk x M column-major, i.e. [i][l][o']) = Dbar^T C^T-view, into Y's buffer
        GSDFT_TRY(gemm_cm('T', 'N', W * k, M, k, 1.0, w.Dfull, dblock_ld(k), w.Cp,
                          padded_cols(k), 0.0, w.Y, W * k, s));
        profile_end(kProfExchGemm, s);
        // Tbar (ld Pc) into the block's buffer: on a symmetric list Dbar_P is symmetric, so the
        // entries of a group, (i, k) and (k, i) and their repeats, share (C Dbar_P C^T)[i][k]:
        // one row per group, over the group CSR; otherwise one row per entry, at its key-order
        // position
        if (sym)
            GSDFT_TRY(launch_sddmm(M, W, k, Pc, w.gptr, w.giota, w.gcol, w.giota, w.Y, w.Cp, w.Bt,
                                   s));
        else
            GSDFT_TRY(launch_sddmm(M, W, k, Pc, row_ptr, row_perm, w.row_col, w.tc.ent_pos, w.Y,
                                   w.Cp, w.Bt, s));
        GSDFT_TRY(exch_tc_reverse(N, q0, W, n, sym ? (n + 1) / 2 : n, w.Bt, Pc, sym, q0 == 0,
                                  w.tc, s));
    }
    GSDFT_TRY(exch_tc_finish(M, n, pi, pj, weight, quat, log_scale, centers, row_ptr,
                             row_perm, col_ptr, col_perm, dquat, dlog_scale, dcenters, w.tc, s));
    return GSDFT_OK;
}
