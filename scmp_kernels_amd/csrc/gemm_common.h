// Definitions shared by the SC GEMM kernels (int8 and FP4 MFMA).
#pragma once

#include "common.h"

namespace scmp {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef char v16c __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Launch parameters of the MFMA SC GEMM kernels (passed by value).
struct GemmP {
    const uint8_t *ca;
    int64_t lda, bsa;
    const uint8_t *cb;
    int64_t ldb, bsb;
    int N, M, D;
    int chunk;
    const int8_t *lut;
    const int32_t *d_class;
    int bipolar;
    scmp_epilogue epi;
    float *y;
    int32_t *iout;
    int64_t ldy, bsy;
    int tilesA, tilesB;
    int nclass;
    // persistent FP4 schedule: ntiles = tilesA * tilesB * batch tiles of 256 x 256, nwg
    // workgroups; split tiles keep exact partial sums in part (2 slots of 256 x 256 floats
    // per workgroup) and count contributors in cnt (ntiles ints, zero on entry)
    int64_t ntiles;
    int nwg;
    float *part;
    int *cnt;
    const int64_t *row_map;   // output row of A row n (NULL: n)
};

// Output row of A row n: the caller's row map scatters a row subset in place.
__device__ __forceinline__ int64_t out_row(const int64_t *row_map, int64_t n) {
    return row_map ? row_map[n] : n;
}

// fp32 epilogue of one output element (row n of A, row m of B, batch index) from its
// exact integer accumulator I, in the operation order of the reference path that the
// kind stands for. One IEEE rounding per operation (no contraction).
__device__ __forceinline__ float epilogue_value(const scmp_epilogue &E, float I, int64_t n,
                                                int64_t m, int64_t batch) {
    switch (E.kind) {
    case SCMP_EPI_ROWCOL: {
        // fl(fl(I*c) * fl(sa*sb)): sc/kernels.py:248 then :1707 / :1271 / :1894
        const float raw = __fmul_rn(I, E.c);
        const float s = __fmul_rn(E.sa[batch * E.sa_batch_stride + n],
                                  E.sb[batch * E.sb_batch_stride + m]);
        return __fmul_rn(raw, s);
    }
    case SCMP_EPI_SCALAR:  // sc/kernels.py:1204 (the scale product is a float64 value)
        return __fmul_rn(__fmul_rn(I, E.c), E.s[0]);
    case SCMP_EPI_HEAD:    // sc/kernels.py:430-432
        return __fmul_rn(I, __fmul_rn(E.c, E.s[batch]));
    case SCMP_EPI_ZP_ROWCOL: {  // sc/kernels.py:1699-1707
        const int64_t na = batch * E.sa_batch_stride + n;
        const int64_t mb = batch * E.sb_batch_stride + m;
        float raw = __fmul_rn(I, E.c);
        const float za = E.za[na], zb = E.zb[mb];
        const float t1 = __fmul_rn(-zb, E.suma[na]);
        const float t2 = __fmul_rn(za, E.sumb[mb]);
        const float t3 = __fmul_rn(__fmul_rn(E.dfloat, za), zb);
        const float corr = __fadd_rn(__fsub_rn(t1, t2), t3);
        raw = __fadd_rn(raw, corr);
        return __fmul_rn(raw, __fmul_rn(E.sa[na], E.sb[mb]));
    }
    default: {  // SCMP_EPI_ZP_SCALAR, sc/kernels.py:1198-1204
        float raw = __fmul_rn(I, E.c);
        const float t1 = __fmul_rn(-E.zb[0], E.suma[batch * E.sa_batch_stride + n]);
        const float t2 = __fmul_rn(E.za[0], E.sumb[batch * E.sb_batch_stride + m]);
        const float corr = __fadd_rn(__fsub_rn(t1, t2), E.t3[0]);
        raw = __fadd_rn(raw, corr);
        return __fmul_rn(raw, E.s[0]);
    }
    }
}

int run_epilogue(const int32_t *iin, float *y, int64_t N, int64_t M, int64_t batch,
                 int64_t ldy, int64_t bsy, const scmp_epilogue &E, const int64_t *row_map,
                 hipStream_t stream);

// FP4 kernel launchers, one translation unit per table width JPF (gemm_fp4_jp*.hip).
// Non-chunked launches apply the epilogue in the kernel (y, or iout for SCMP_EPI_INT).
template <int JPF>
int gemm_fp4_launch_jpf(const GemmP &P, int64_t batch, bool chunked, hipStream_t stream);
int gemm_fp4_run(GemmP &P, const scmp_gemm_args &a, bool chunked, hipStream_t stream);

}  // namespace scmp
