// Lane orders of the three-centre passes.
//
// Forward (one lane per aux function):
// Aux functions are sorted by an exponent band (a factor 4 in b = e^log_alpha) and then by the
// Morton code of their centre on a 1-Bohr grid (+-256 Bohr, clamped), so that the 64 functions of
// a wave are close in space and in width and the node screen of the forward kernel fires for
// whole waves. The order only decides which functions share a wave: each function's own sum runs
// over the pairs in the same sequence whatever its lane. A stable radix sort of 31-bit keys makes
// the order a pure function of the inputs.
#include <hipcub/hipcub.hpp>

#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

__device__ __forceinline__ uint32_t spread3(uint32_t v) {   // 9 bits -> every third of 27
    v &= 0x1ff;
    v = (v | (v << 16)) & 0x030000ff;
    v = (v | (v << 8)) & 0x0300f00f;
    v = (v | (v << 4)) & 0x030c30c3;
    v = (v | (v << 2)) & 0x09249249;
    return v;
}

__global__ void k_aux_keys(int64_t N, const double* __restrict__ log_alpha,
                           const double* __restrict__ R, uint32_t* __restrict__ key,
                           int32_t* __restrict__ idx) {
    const int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (p >= N) return;
    // fmin/fmax return the number when the other operand is NaN, so every key is defined.
    const double band = __builtin_fmax(__builtin_fmin(
        __builtin_floor(log_alpha[p] * 0x1.71547652b82fep-1) + 8.0, 15.0), 0.0);   // log4 b + 8
    uint32_t code = 0;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const double c = __builtin_fmax(__builtin_fmin(__builtin_floor(R[3 * p + d] + 256.0),
                                                       511.0), 0.0);
        code |= spread3((uint32_t)c) << d;
    }
    key[p] = ((uint32_t)band << 27) | code;
    idx[p] = (int32_t)p;
}

__device__ __forceinline__ uint64_t spread3_10(uint32_t v) {   // 10 bits -> every third of 30
    uint64_t x = v & 0x3ff;
    x = (x | (x << 16)) & 0x30000ffull;
    x = (x | (x << 8)) & 0x300f00full;
    x = (x | (x << 4)) & 0x30c30c3ull;
    x = (x | (x << 2)) & 0x9249249ull;
    return x;
}

// rec: pair records in list order (I1 I2 I3 | Ah | P | ...), stride rec_stride doubles.
__global__ void k_pair_keys(int64_t n, const double* __restrict__ rec, int rec_stride,
                            uint64_t* __restrict__ key, int32_t* __restrict__ idx) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    const double* r = rec + (int64_t)rec_stride * a;
    const double band = __builtin_fmax(__builtin_fmin(
        __builtin_floor(0.5 * log2(r[2] / r[1])) + 8.0, 15.0), 0.0);
    uint64_t code = 0;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
        const double c = __builtin_fmax(__builtin_fmin(__builtin_floor(2.0 * (r[9 + d] + 256.0)),
                                                       1023.0), 0.0);
        code |= spread3_10((uint32_t)c) << d;
    }
    key[a] = ((uint64_t)band << 30) | code;
    idx[a] = (int32_t)a;
}

}  // namespace

int pair_order_layout(Arena& ar, int64_t n, PairOrderWs* w) {
    w->key_in = ar.take<uint64_t>(n + 1);
    w->key_out = ar.take<uint64_t>(n + 1);
    w->idx_in = ar.take<int32_t>(n + 1);
    w->perm = ar.take<int32_t>(n + 1);
    w->sort_bytes = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, w->sort_bytes, (const uint64_t*)nullptr,
                                           (uint64_t*)nullptr, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)(n > 0 ? n : 1), 0, 34) !=
        hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub sort size query failed");
    w->sort_tmp = ar.take<char>(w->sort_bytes);
    return GSDFT_OK;
}

int launch_pair_order(int64_t n, const double* rec, int rec_stride, const PairOrderWs& w,
                      hipStream_t s) {
    if (n > INT32_MAX) return fail(GSDFT_ERR_ARG, "pair order: n exceeds the int32 range");
    if (n <= 0) return GSDFT_OK;
    k_pair_keys<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(n, rec, rec_stride, w.key_in,
                                                            w.idx_in);
    GSDFT_HIP(hipGetLastError());
    size_t b = w.sort_bytes;
    GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(w.sort_tmp, b, w.key_in, w.key_out, w.idx_in,
                                                 w.perm, (int)n, 0, 34, s));
    return GSDFT_OK;
}

int aux_order_layout(Arena& ar, int64_t N, AuxOrderWs* w) {
    w->key_in = ar.take<uint32_t>(N + 1);
    w->key_out = ar.take<uint32_t>(N + 1);
    w->idx_in = ar.take<int32_t>(N + 1);
    w->order = ar.take<int32_t>(N + 1);
    w->sort_bytes = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, w->sort_bytes, (const uint32_t*)nullptr,
                                           (uint32_t*)nullptr, (const int32_t*)nullptr,
                                           (int32_t*)nullptr, (int)N, 0, 31) != hipSuccess)
        return fail(GSDFT_ERR_LIB, "hipcub sort size query failed");
    w->sort_tmp = ar.take<char>(w->sort_bytes);
    return GSDFT_OK;
}

int launch_aux_order(int64_t N, const double* log_alpha, const double* aux_centers,
                     const AuxOrderWs& w, hipStream_t s) {
    if (N > INT32_MAX) return fail(GSDFT_ERR_ARG, "aux order: N exceeds the int32 range");
    k_aux_keys<<<(unsigned)((N + 255) / 256), 256, 0, s>>>(N, log_alpha, aux_centers, w.key_in,
                                                           w.idx_in);
    GSDFT_HIP(hipGetLastError());
    size_t b = w.sort_bytes;
    GSDFT_HIP(hipcub::DeviceRadixSort::SortPairs(w.sort_tmp, b, w.key_in, w.key_out, w.idx_in,
                                                 w.order, (int)N, 0, 31, s));
    return GSDFT_OK;
}

}  // namespace gsdft
