// Definitions shared by the SC GEMM kernels (int8 and FP4 MFMA).
#pragma once

#include "common.h"

namespace scmp {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef char v16c __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

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
    int JP;                   // intervals per table row (16 .. 256)
    scmp_epilogue epi;
    float *y;
    int32_t *iout;
    int64_t ldy, bsy;
    int tilesA, tilesB;
    int nclass;
    // persistent FP4 schedule: ntiles = tilesA * tilesB * batch tiles of 256 x tile_cols
    // (256, or 64 for narrow outputs), nwg workgroups; split tiles keep exact partial sums
    // in part (2 slots of one tile's floats per workgroup) and count contributors in cnt
    // (ntiles ints, zero on entry)
    int tile_cols;
    int64_t ntiles;
    int nwg;                  // persistent workgroups (chunked launch: compute units)
    float *part;
    int *cnt;
    const int64_t *row_map;   // output row of A row n (NULL: n)
    const int32_t *group_class;   // FP4: class of each 8-d group (NULL: none)
    int row0;                 // chunked FP4 launch: first A row it computes
    // FP4 split tiles: 0 = the last contributor to arrive adds the others' partial sums and
    // applies the epilogue; 1 = every contributor publishes its partial sums and a fixup
    // launch after the GEMM finishes the shared tiles (no counters)
    int deferred;
};

// Output row of A row n: the caller's row map scatters a row subset in place.
__device__ __forceinline__ int64_t out_row(const int64_t *row_map, int64_t n) {
    return row_map ? row_map[n] : n;
}

// fp32 epilogue of one output element from its exact integer accumulator I, in the
// operation order of the reference path that the kind stands for. One IEEE rounding per
// operation (no contraction). The inputs split into row factors (sa, za, suma of row n),
// column factors (sb, zb, sumb of column m) and tile-uniform values (s, za, zb, t3 of the
// scalar kinds), so a kernel can load them once per tile instead of once per element.
struct EpiUniform {
    float s, za, zb, t3;
};

__device__ __forceinline__ EpiUniform epi_uniform(const scmp_epilogue &E, int64_t batch) {
    EpiUniform u = {0.f, 0.f, 0.f, 0.f};
    if (E.kind == SCMP_EPI_SCALAR) u.s = E.s[0];
    else if (E.kind == SCMP_EPI_HEAD)   // s[batch], or the head's two scales' fp32 product
        u.s = E.s ? E.s[batch]
                  : __fmul_rn(E.sa[batch * E.sa_batch_stride], E.sb[batch * E.sb_batch_stride]);
    else if (E.kind == SCMP_EPI_ZP_SCALAR) {
        u.s = E.s[0];
        u.za = E.za[0];
        u.zb = E.zb[0];
        u.t3 = E.t3[0];
    }
    return u;
}

// f[0..2] = sa, za, suma of row n (only those the kind reads)
__device__ __forceinline__ void epi_row_factors(const scmp_epilogue &E, int64_t n, int64_t batch,
                                                float (&f)[3]) {
    const int64_t i = batch * E.sa_batch_stride + n;
    f[0] = f[1] = f[2] = 0.f;
    if (E.kind == SCMP_EPI_ROWCOL || E.kind == SCMP_EPI_ZP_ROWCOL) f[0] = E.sa[i];
    if (E.kind == SCMP_EPI_ZP_ROWCOL) f[1] = E.za[i];
    if (E.kind == SCMP_EPI_ZP_ROWCOL || E.kind == SCMP_EPI_ZP_SCALAR) f[2] = E.suma[i];
}

// f[0..2] = sb, zb, sumb of column m (only those the kind reads)
__device__ __forceinline__ void epi_col_factors(const scmp_epilogue &E, int64_t m, int64_t batch,
                                                float (&f)[3]) {
    const int64_t i = batch * E.sb_batch_stride + m;
    f[0] = f[1] = f[2] = 0.f;
    if (E.kind == SCMP_EPI_ROWCOL || E.kind == SCMP_EPI_ZP_ROWCOL) f[0] = E.sb[i];
    if (E.kind == SCMP_EPI_ZP_ROWCOL) f[1] = E.zb[i];
    if (E.kind == SCMP_EPI_ZP_ROWCOL || E.kind == SCMP_EPI_ZP_SCALAR) f[2] = E.sumb[i];
}

template <int KIND>
__device__ __forceinline__ float epilogue_apply_k(const scmp_epilogue &E, float I, float ra,
                                                  float rz, float rs, float cb, float cz,
                                                  float cs, const EpiUniform &u) {
    if constexpr (KIND == SCMP_EPI_ROWCOL) {
        // fl(fl(I*c) * fl(sa*sb)): sc/kernels.py:248 then :1707 / :1271 / :1894
        return __fmul_rn(__fmul_rn(I, E.c), __fmul_rn(ra, cb));
    } else if constexpr (KIND == SCMP_EPI_SCALAR) {
        // sc/kernels.py:1204 (the scale product is a float64 value)
        return __fmul_rn(__fmul_rn(I, E.c), u.s);
    } else if constexpr (KIND == SCMP_EPI_HEAD) {
        return __fmul_rn(I, __fmul_rn(E.c, u.s));           // sc/kernels.py:430-432
    } else if constexpr (KIND == SCMP_EPI_ZP_ROWCOL) {      // sc/kernels.py:1699-1707
        float raw = __fmul_rn(I, E.c);
        const float t1 = __fmul_rn(-cz, rs);
        const float t2 = __fmul_rn(rz, cs);
        const float t3 = __fmul_rn(__fmul_rn(E.dfloat, rz), cz);
        raw = __fadd_rn(raw, __fadd_rn(__fsub_rn(t1, t2), t3));
        return __fmul_rn(raw, __fmul_rn(ra, cb));
    } else {                                                // SCMP_EPI_ZP_SCALAR, :1198-1204
        float raw = __fmul_rn(I, E.c);
        const float t1 = __fmul_rn(-u.zb, rs);
        const float t2 = __fmul_rn(u.za, cs);
        raw = __fadd_rn(raw, __fadd_rn(__fsub_rn(t1, t2), u.t3));
        return __fmul_rn(raw, u.s);
    }
}

__device__ __forceinline__ float epilogue_apply(const scmp_epilogue &E, float I, float ra,
                                                float rz, float rs, float cb, float cz,
                                                float cs, const EpiUniform &u) {
    switch (E.kind) {
    case SCMP_EPI_ROWCOL: return epilogue_apply_k<SCMP_EPI_ROWCOL>(E, I, ra, rz, rs, cb, cz, cs, u);
    case SCMP_EPI_SCALAR: return epilogue_apply_k<SCMP_EPI_SCALAR>(E, I, ra, rz, rs, cb, cz, cs, u);
    case SCMP_EPI_HEAD: return epilogue_apply_k<SCMP_EPI_HEAD>(E, I, ra, rz, rs, cb, cz, cs, u);
    case SCMP_EPI_ZP_ROWCOL:
        return epilogue_apply_k<SCMP_EPI_ZP_ROWCOL>(E, I, ra, rz, rs, cb, cz, cs, u);
    default: return epilogue_apply_k<SCMP_EPI_ZP_SCALAR>(E, I, ra, rz, rs, cb, cz, cs, u);
    }
}

// The epilogue of one element, loading its factors (kernels without per-tile staging).
__device__ __forceinline__ float epilogue_value(const scmp_epilogue &E, float I, int64_t n,
                                                int64_t m, int64_t batch) {
    float r[3], c[3];
    epi_row_factors(E, n, batch, r);
    epi_col_factors(E, m, batch, c);
    return epilogue_apply(E, I, r[0], r[1], r[2], c[0], c[1], c[2], epi_uniform(E, batch));
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
