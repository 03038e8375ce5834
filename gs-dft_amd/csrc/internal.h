// Host-side launchers shared between the translation units of libgsdft.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/gsdft.h"
#include "common.h"

namespace gsdft {

// Error reporting: a thread-local message behind gsdft_last_error().
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);

#define GSDFT_HIP(call)                                                   \
    do {                                                                  \
        hipError_t e_ = (call);                                           \
        if (e_ != hipSuccess) return ::gsdft::hip_fail(e_, #call);        \
    } while (0)

#define GSDFT_TRY(call)                                                   \
    do {                                                                  \
        int rc_ = (call);                                                 \
        if (rc_ != GSDFT_OK) return rc_;                                  \
    } while (0)

// One dimension of a grid holds at most 2^32 - 1 work-items. The one-dimensional launches over a
// pair list take at most 25 work-items per pair (the reverse's moments), so every entry point that
// takes a list accepts at most kMaxPairs pairs and reports larger ones rather than launching a
// grid whose size would wrap.
constexpr int64_t kMaxPairs = 160000000;
// Element-wise launches over a dense array use one work-item per element: the arrays they cover
// must stay within one grid dimension.
constexpr int64_t kMaxLaunchItems = (int64_t)UINT32_MAX - 255;
inline int check_items(int64_t items, const char* who, const char* what) {
    return items > kMaxLaunchItems
               ? fail(GSDFT_ERR_ARG, "%s: %s has %lld elements, more than one launch covers (%lld)",
                      who, what, (long long)items, (long long)kMaxLaunchItems)
               : GSDFT_OK;
}
inline int check_pairs(int64_t n, const char* who) {
    return n > kMaxPairs ? fail(GSDFT_ERR_ARG, "%s: n = %lld pairs, more than the %lld one call takes",
                                who, (long long)n, (long long)kMaxPairs)
                         : GSDFT_OK;
}

// Bump allocator over a caller-provided workspace (256-byte aligned slices).
struct Arena {
    char* base;
    size_t cap;
    size_t used;
    template <class T>
    T* take(size_t count) {
        size_t off = (used + 255) & ~size_t(255);
        used = off + count * sizeof(T);
        return (base && used <= cap) ? reinterpret_cast<T*>(base + off) : nullptr;
    }
    size_t need() const { return (used + 255) & ~size_t(255); }
};

// Copies `bytes` from device memory into host memory and waits on stream s before returning,
// whatever the outcome, so no copy into the host buffer (often a stack local) is ever left in
// flight behind an early return.
int read_back(void* host, const void* dev, size_t bytes, hipStream_t s, const char* what);

// Optional per-kernel timing with HIP events on the launch stream.
void profile_begin(int id, hipStream_t s);
void profile_end(int id, hipStream_t s);
// Brackets a scope with profile_begin / profile_end, so every return path closes the interval.
struct ProfileScope {
    int id;
    hipStream_t s;
    ProfileScope(int id_, hipStream_t s_) : id(id_), s(s_) { profile_begin(id, s); }
    ~ProfileScope() { profile_end(id, s); }
    ProfileScope(const ProfileScope&) = delete;
    ProfileScope& operator=(const ProfileScope&) = delete;
};
// Device counter of work units for kernel id while profiling is on (current device only), else
// nullptr; kernels given a counter add their executed units to it.
unsigned long long* profile_work_counter(int id);
enum ProfileId { kProfGammaFwd = 0, kProfGammaBwd = 1, kProfScreen = 2, kProfMetric = 3,
                 kProfCholesky = 4, kProfSolve = 5, kProfNucPairs = 6, kProfNucAtoms = 7,
                 kProfEriFwd = 8, kProfEriBwd = 9, kProfExchBlock = 10, kProfExchBwd = 11,
                 kProfExchTrsm = 12, kProfExchGemm = 13, kProfExchSparse = 14,
                 kProfCount = 15 };

// gemm.hip: C(m, n) -= sum_k A[m lda + k] B[n ldb + k] for m < Mr, n < Nc (C column-major,
// C(m, n) at C[n ldc + m]) on FP64 MFMA; with `upper` (Mr == Nc) only the 128 x 128 tiles on or
// above the diagonal are formed (the diagonal tiles in full).
int launch_gemm_tn_sub(int64_t Mr, int64_t Nc, int64_t K, const double* A, int64_t lda,
                       const double* B, int64_t ldb, double* C, int64_t ldc, bool upper,
                       hipStream_t s);

// gemm.hip: C = alpha op(A) op(B) + beta C over Mr x Nc (C column-major, leading dimension ldc;
// beta = 0 does not read C), op(A)(m, k) at A[m lda + k] when a_kc (k-contiguous), else at
// A[k lda + m]; op(B)(k, n) at B[n ldb + k] when b_kc, else at B[k ldb + n]; `batch` products
// with the operands `stride_*` doubles apart. FP64 MFMA tiles of 128 x 128.
int launch_gemm(int64_t Mr, int64_t Nc, int64_t K, double alpha, const double* A, int64_t lda,
                bool a_kc, int64_t stride_a, const double* B, int64_t ldb, bool b_kc,
                int64_t stride_b, double beta, double* C, int64_t ldc, int64_t stride_c,
                int64_t batch, hipStream_t s);

// The same as a column-major BLAS dgemm: C (m x n) = alpha op(A) op(B) + beta C, op = 'N' or 'T'.
int gemm_cm(char transa, char transb, int64_t m, int64_t n, int64_t k, double alpha,
            const double* A, int64_t lda, const double* B, int64_t ldb, double beta, double* C,
            int64_t ldc, hipStream_t s);

// gemm_cm with K split over S = gemm_split_slices(m, n, k) slices when the m x n output has too
// few tiles to fill the GPU (fewer when part, part_doubles long, holds fewer m x n blocks): the
// slices' products go to part (column-major m x n each) and are added in slice order,
// C = alpha op(A) op(B) + beta C; with S = 1 it is gemm_cm.
int64_t gemm_split_slices(int64_t m, int64_t n, int64_t k);
int gemm_cm_split(char transa, char transb, int64_t m, int64_t n, int64_t k, double alpha,
                  const double* A, int64_t lda, const double* B, int64_t ldb, double beta,
                  double* C, int64_t ldc, double* part, int64_t part_doubles, hipStream_t s);
// The same with the caller's slice count S (part holds S m x n blocks; slices of (k / S) rounded
// down to a multiple of 16, the remainder joining the last one); gemm_cm when S <= 1 or k < 16 S.
int gemm_cm_slices(char transa, char transb, int64_t m, int64_t n, int64_t k, double alpha,
                   const double* A, int64_t lda, const double* B, int64_t ldb, double beta,
                   double* C, int64_t ldc, int64_t S, double* part, hipStream_t s);

// dfj.hip: X (m x n, column-major, leading dimension ldx) <- X U^-1 (X U = B) or, with trans,
// X U^-T (X U^T = B), for the n x n upper U (column-major, leading dimension ldu), by blocked
// substitution with FP64 MFMA products between the blocks; `part` (part_doubles long, may be
// null) holds the K-slices of the products whose output has too few tiles to fill the GPU.
int trsm_right_upper(hipStream_t s, bool trans, int64_t n, const double* U, int64_t ldu,
                     double* X, int64_t m, int64_t ldx, double* part = nullptr,
                     int64_t part_doubles = 0);

// solve.hip: forward then backward substitution with the row-major lower factor, in place.
int launch_trsv_pair(int64_t N, const double* L, double* x, hipStream_t s);

// order.hip: slot order of the three-centre passes (perm[slot] = pair index), built from
// pair records in list order whose first 12 doubles are I1 I2 I3 | Ah (6) | P (3).
struct PairOrderWs {
    uint64_t *key_in, *key_out;
    int32_t *idx_in, *perm;
    char* sort_tmp;
    size_t sort_bytes;
};
int pair_order_layout(Arena& ar, int64_t n, PairOrderWs* w);
// With n_live (a device count), only the first *n_live records are real: the rest take the slots
// after them.
int launch_pair_order(int64_t n, const double* rec, int rec_stride, const PairOrderWs& w,
                      hipStream_t s, const int64_t* n_live = nullptr);
// order.hip: groups of list entries by unordered splat pair and weight (live entries with equal
// weights q; each dead entry, q = 0, alone), numbered in key order, through the sort buffers of po
// (sized for n). Fills ent_group and ent_pos (per entry), grp_first (n_groups + 1) and grp_rep
// (per group) and the device count *n_groups; head is n ints of scratch, scan_tmp
// pair_groups_scan_bytes(n) bytes.
size_t pair_groups_scan_bytes(int64_t n);
int launch_pair_groups(int64_t M, int64_t n, const int32_t* pi, const int32_t* pj,
                       const double* q, const PairOrderWs& po, int32_t* head, char* scan_tmp,
                       size_t scan_bytes, int32_t* ent_group, int32_t* ent_pos,
                       int32_t* grp_first, int32_t* grp_rep, int64_t* n_groups, hipStream_t s);

// dfj.hip: the three-centre passes of the screened exchange. Charts, aux quantities and pair
// records (q_a = w_a) in list order. The entries of the list are grouped by their unordered splat
// pair {i, j} (live entries only; each dead entry is a group of its own): the entries of a group
// share one product Gaussian and so one (P|a), which the passes form once per group. Groups are
// numbered in order of their first entry in key order; per entry its group (ent_group) and its
// position in key order (ent_pos, the row of its cotangent), per group its first key-order
// position (grp_first, n_groups + 1 entries) and its first entry (grp_rep). The three-centre
// passes run over the groups in slot order (pair_order.perm: slot -> group); slot_pair maps a
// slot to its group's first entry.
struct ExchTcWs {
    double *A6, *Nrm, *beta, *kn, *q, *rec;
    double *rec_grp, *rec_sorted, *aux, *part, *acc, *J, *contrib;
    int32_t *ent_group, *ent_pos, *grp_first, *grp_rep, *slot_pair, *head;
    int64_t* n_groups_dev;
    char* scan_tmp;
    size_t scan_bytes;
    PairOrderWs pair_order;
    NodeTable table;        // the kernel's node rule (set after exch_tc_layout)
};
// The node rule of the 1/r kernel and of the long-range erf(omega r)/r kernel (omega > 0).
NodeTable coulomb_table();
NodeTable long_range_table(double omega);
int exch_tc_layout(Arena& ar, int64_t M, int64_t N, int64_t n, int64_t Pc, bool grads,
                   ExchTcWs* w);
// Charts, records, the groups and their slot order. The group count stays on the device
// (n_groups_dev; nothing is read back): the passes below run over n slots, the first
// *n_groups_dev of them the groups, the rest idle.
int exch_tc_prologue(int64_t M, const double* quat, const double* log_scale,
                     const double* centers, int64_t N, const double* log_alpha,
                     const double* aux_centers, int64_t n, const int32_t* pi, const int32_t* pj,
                     const double* weight, bool grads, const ExchTcWs& w, hipStream_t s);
// Bt[g * ldb + l] = (P|a) w_g for every group g and the aux of slots q0 .. q0 + W - 1 (slot order:
// the G = N / M scales of one centre consecutive when N is a multiple of M, else aux order).
int exch_tc_block(int64_t M, int64_t N, int64_t q0, int64_t W, const double* aux_centers,
                  int64_t n, int64_t ldb, double* Bt, const ExchTcWs& w, hipStream_t s);
// Adds (first: sets) the reverse moments of the aux slots q0 .. q0 + W - 1 with the cotangent of
// group g's (P|a_l): the sum, in key order, of Tbar[e * ldt + l] over its entries' key-order
// positions e; with group_rows, Tbar[g * ldt + l] (the entries' common cotangent) times the
// group's entry count. n_est (at least n / 2) estimates the group count for the split of the aux
// slots.
int exch_tc_reverse(int64_t N, int64_t q0, int64_t W, int64_t n, int64_t n_est,
                    const double* Tbar, int64_t ldt, bool group_rows, bool first,
                    const ExchTcWs& w, hipStream_t s);
// Moments -> per-group splat contributions (on the group's first entry, zero on the others) ->
// dquat, dlog_scale, dcenters.
int exch_tc_finish(int64_t M, int64_t n, const int32_t* pi, const int32_t* pj,
                   const double* weight, const double* quat, const double* log_scale,
                   const double* centers, const int32_t* row_ptr, const int32_t* row_perm,
                   const int32_t* col_ptr, const int32_t* col_perm, double* dquat,
                   double* dlog_scale, double* dcenters, const ExchTcWs& w, hipStream_t s);

// screen.hip
int launch_chart(int64_t M, const double* quat, const double* log_scale, double* A6, double* N,
                 hipStream_t s);

}  // namespace gsdft
