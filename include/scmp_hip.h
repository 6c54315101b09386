/*
 * scmp_hip.h -- C ABI of libscmp_hip.so, the MI355X (gfx950) implementation of the
 * stochastic-computing (SC) matmul path of swalther06/scmp_kernels.
 *
 * Conventions
 *  - All pointers are device pointers unless a comment says "host".
 *  - Every call is asynchronous and stream-ordered on the hipStream_t argument; none
 *    synchronizes the host. The library allocates no device memory: callers pass every
 *    output and workspace buffer.
 *  - Return value: 0 on success, a negative SCMP_E* code on invalid arguments or a HIP
 *    launch error; scmp_last_error() then describes it (thread-local string).
 *  - The entry points are stateless and reentrant.
 *
 * Each entry point names the reference interface it replaces (paths relative to the
 * reference repository root).
 */
#ifndef SCMP_HIP_H
#define SCMP_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SCMP_OK 0
#define SCMP_E_ARG (-1)
#define SCMP_E_LAUNCH (-2)
#define SCMP_E_UNSUPPORTED (-3)

/* Library identification and the last error message of the calling thread. Version 2:
 * scmp_quant_args.row_index, scmp_gemm_args.row_map and scmp_gemm_args.group_class;
 * version 3: scmp_quant_args.given_absmax. */
int scmp_abi_version(void);
const char *scmp_last_error(void);

/* ---------------------------------------------------------------------------------
 * RNG sequences
 * ------------------------------------------------------------------------------- */

/* Gray-code Sobol sequence of n values from p direction vectors (host array V[p]).
 * Replaces Sobol.simulate, scmp_kernels/sc/rng.py:185-225. */
int scmp_rng_sobol(int p, const int64_t *V_host, int64_t n, int32_t *out, hipStream_t stream);

/* Fibonacci right-shift LFSR sequence (output = register, then shift in the XOR of the
 * bits selected by taps_mask at bit length-1). Replaces LFSR.simulate,
 * scmp_kernels/sc/rng.py:55-77. */
int scmp_rng_lfsr(int length, int64_t seed, uint64_t taps_mask, int64_t n, int32_t *out,
                  hipStream_t stream);

/* Per-element sequences: out[d, t] = scramble(base[src[d], t], perm[d]) for d < D.
 * perm: D x p bit permutations (output bit i <- input bit perm[d*p+i]); a row whose first
 * entry is -1 is copied unchanged; perm may be NULL (no scrambles at all).
 * Replaces SNGBank.get_all_sequences / apply_scramble(_batch),
 * scmp_kernels/sc/sng.py:15-53, 187-230. */
int scmp_rng_expand(const int32_t *base, int64_t n, const int32_t *src, const int32_t *perm,
                    int p, int D, int32_t *out, hipStream_t stream);

/* LFSR tap-set search for an n_bits register (2 <= n_bits <= SCMP_LFSR_SEARCH_MAX_BITS):
 * distinct[i] = number of distinct states the right-shift LFSR with tap bit mask masks[i]
 * visits from seed 1 before its first repeat (a tap set is maximal-length when this is
 * 2^n_bits - 1). One device thread per candidate (Brent cycle detection, O(1) state).
 * Replaces _is_maximal_length and the enumeration loop of search_taps,
 * scmp_kernels/sc/lfsr_taps.py:35-111. */
#define SCMP_LFSR_SEARCH_MAX_BITS 20
int scmp_lfsr_search(int n_bits, const uint32_t *masks, int64_t count, uint32_t *distinct,
                     hipStream_t stream);

/* Prefix / Owen XOR / rescale: out[d, t] for t < L from r[d, t] (row length full).
 * masks: per-d XOR masks or NULL (Owen off). R == 2^p: XOR only when L < full.
 * Otherwise XOR when scramble_rescale, then floor(v * R / 2^p).
 * Replaces _prepare_rng_prefix / _owen_scramble, scmp_kernels/sc/kernels.py:646-704. */
int scmp_rng_prepare(const int32_t *r, int D, int full, int p, int L, int R,
                     const int32_t *masks, int scramble_rescale, int32_t *out,
                     hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Stream tables for the SC GEMM (replaces build_cum_indicator_kernel and
 * compute_k_table_kernel, scmp_kernels/sc/kernels.py:102-169, 712-759).
 *
 * For each table class c (one class per distinct pair of A/B sequences; rep[c] is a
 * dimension d of that class) with A-side sequence ra[rep] and B-side sequence rb[rep]
 * (both length L, values already prepared), and the boundary map
 * beta(q) = rne(fl(fl(q*R)/Q)):
 *   K(v)      = #{t < L : ra[t] < v}
 *   kappa_0 < kappa_1 < ... < kappa_J   distinct values of K(beta(q)), q = 0..qmax
 *   jtab[c][q] = j with kappa_j = K(beta(q))               (q = |code| index, 256 entries)
 *   lut[c][row][byte 4u+b] = s * #{i in [kappa_j', kappa_j'+1) : rb[i] < beta(|q|)}
 *                           for j' = (JP/4)*b + u, row = code byte of q, s = sign(q)
 *   kappa[c][j] (int16, JP+1 entries)
 * bipolar: Q = 2^(p-1)-1, codes are int8 q in [-(Q+1), Q]; unipolar: Q = 2^p-1,
 * codes are uint8 q in [0, Q]. JP (16..256, power of two) must be >= every class's J.
 * Returns SCMP_E_ARG if some class needs J > JP. */
int scmp_build_stream_tables(const int32_t *ra, const int32_t *rb, const int32_t *rep,
                             int nclass, int L, int p, int R, int bipolar, int JP,
                             uint8_t *jtab, int8_t *lut, int16_t *kappa, int32_t *jmax_out,
                             hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * Quantizers (replace fused_quant_kernel / fused_quant_bipolar_batched_kernel,
 * scmp_kernels/quant/fused.py:35-283, and the torch row-group quantizers,
 * scmp_kernels/quant/grouped.py:13-163)
 * ------------------------------------------------------------------------------- */

/* Quantizer variants (fp32 operation order of each is that of its reference) */
#define SCMP_Q_GROUP_SYM 0    /* _grouped_symmetric_quant: q = rne(x / s), zero sign +1 */
#define SCMP_Q_ROW_SYM 1      /* fused per-row: q = rne(x * fl(1/s)), zero sign 0 */
#define SCMP_Q_TENSOR_SYM 2   /* fused per-tensor: float64 host-style scale, zero sign 0 */
#define SCMP_Q_HEAD_SYM 3     /* fused batched per-head: clamp [-(Q+1), Q], zero sign 0 */
#define SCMP_Q_GROUP_ASYM 4   /* _grouped_asymmetric_quant: q = rne(fl(x / s) + zp) */
#define SCMP_Q_TENSOR_ASYM 5  /* fused per-tensor unipolar (float64 scale/zp) */
#define SCMP_Q_HOST_SYM 6     /* fused flat bipolar with the caller's fp32 reciprocal */
#define SCMP_Q_HOST_ASYM 7    /* fused unipolar with the caller's fp32 reciprocal and zp */

/* SmoothQuant fused into the load (apply_smoothing, scmp_kernels/quant/smoothquant.py:
 * 124-126): x' = fl(x / s[col]) (DIV) or fl(x * s[col]) (MUL). */
#define SCMP_SMOOTH_NONE 0
#define SCMP_SMOOTH_DIV 1
#define SCMP_SMOOTH_MUL 2

/* Code outputs for the SC GEMM */
#define SCMP_CODE_NONE 0
#define SCMP_CODE_THERMO 1    /* A side: (sign bit 7) | jtab[class(col)][|q|] */
#define SCMP_CODE_Q 2         /* B side: q as a byte */

typedef struct scmp_quant_args {
    /* input: rows x cols fp32, row stride ld (elements) */
    const float *x;
    int64_t rows, cols, ld;
    const float *smooth;      /* (cols,) or NULL */
    int smooth_mode;
    int variant;              /* SCMP_Q_* */
    int64_t group;            /* rows per group (>= rows: one group) */
    int64_t seg;              /* columns per segment (chunk_d); 0 = whole row */
    int q_max;                /* Q (<= 255 when codes are written) */
    int rng_levels;           /* R, for the boundary outputs */
    float host_inv, host_zp;  /* HOST_* variants: reciprocal scale and zero-point */
    /* GEMM codes: the input rows form batches of code_batch_rows rows (0: one batch);
     * batch b, row i goes to code[(b * code_rows + i) * code_ld + col]; rows
     * code_batch_rows..code_rows-1 of every batch and columns cols..code_ld-1 are zero;
     * code_ld >= cols rounded up to a multiple of 4 */
    int code_kind;
    uint8_t *code;
    int64_t code_ld, code_rows, code_batch_rows;
    const uint8_t *jtab;      /* THERMO: nclass x 256 */
    const int32_t *col_class; /* THERMO: class of each column, NULL = class 0 */
    /* reference API outputs (each optional) */
    int16_t *beta16;          /* boundary int16 (rows x cols) */
    int32_t *beta32;          /* boundary int32 (unipolar fused API) */
    int beta_formula;         /* 0: rne(|q| * fl32(R/Q)); 1: rne(fl(fl(|q|*R)/Q)) */
    int8_t *sign;             /* sign int8 (rows x cols) */
    float *xint;              /* quantized integers as fp32 (rows x cols) */
    int64_t out_ld;           /* row stride of beta/sign/xint (elements) */
    float *scale;             /* per (row, segment): scale[seg * rows + row] */
    double *scale64;          /* TENSOR variants: float64 scale (one value) */
    float *inv;               /* per (row, segment) fp32 reciprocal actually used, or NULL */
    float *zp;                /* ASYM: per row zero-point (fp32) */
    double *zp64;             /* TENSOR_ASYM: zero-point as float64 */
    float *rowsum;            /* sum of q over the row (exact integers as fp32) */
    /* workspace: >= scmp_quant_workspace_bytes(...) bytes */
    void *workspace;
    /* input row of each quantized row: row r reads x row row_index[r] (each a valid row of
     * x), so a caller quantizes a row subset in any order without gathering it; NULL: r */
    const int64_t *row_index;
    /* symmetric row-group variants (GROUP_SYM, ROW_SYM, HEAD_SYM) without column segments:
     * max|x| of each row group given by the caller, one fp32 per group (non-negative), used
     * in place of the reduction over x (the reference's _sc_matmul_per_head_bipolar takes
     * its per-head ranges as arguments, scmp_kernels/sc/kernels.py:440-495); NULL: reduced */
    const float *given_absmax;
} scmp_quant_args;

int64_t scmp_quant_workspace_bytes(int64_t rows, int64_t cols, int64_t group, int64_t seg);
int scmp_quantize(const scmp_quant_args *args, hipStream_t stream);

/* Two independent quantizer calls, a then b, with the results of two scmp_quantize calls.
 * Replaces the per-head path's two quantizer calls on q and k
 * (scmp_kernels/sc/kernels.py:484-516). When both are SCMP_Q_HEAD_SYM code-only calls of
 * dense rows (16-byte aligned, ld = code_ld = cols, no smoothing, row index or given ranges),
 * a with THERMO codes and no column classes, b with Q codes, and each takes 5 to 16 four-column
 * chunks per thread at 256 threads per row group, both run in one launch. Otherwise they run
 * as two calls. */
int scmp_quantize_pair(const scmp_quant_args *a, const scmp_quant_args *b, hipStream_t stream);

/* ---------------------------------------------------------------------------------
 * SC GEMM (replaces enable_matmul_tiled_kernel / enable_matmul_bipolar_batched_kernel /
 * enable_matmul_compact_dot_kernel, scmp_kernels/sc/kernels.py:176-332, 362-437, and the
 * epilogues at kernels.py:1204, 1271, 1381, 1413-1418, 1699-1707, 1894, 550)
 *
 *   I[n, m] = sum_d sum_{j' < JP} thermo(codes_a[n, d])[j'] * lut[class(d)][codes_b[m, d]][j']
 * ------------------------------------------------------------------------------- */

#define SCMP_EPI_INT 0        /* iout[n, m] = I (int32) */
#define SCMP_EPI_ROWCOL 1     /* fl(fl(I*c) * fl(sa[n]*sb[m])); per chunk, summed in order */
#define SCMP_EPI_SCALAR 2     /* fl(fl(I*c) * s[0]) */
#define SCMP_EPI_HEAD 3       /* fl(I * fl(c * s[batch])); s NULL: s[batch] =
                               * fl(sa[batch * sa_batch_stride] * sb[batch * sb_batch_stride]) */
#define SCMP_EPI_ZP_ROWCOL 4  /* fl(fl(fl(I*c) + corr) * fl(sa*sb)), grouped zero-point */
#define SCMP_EPI_ZP_SCALAR 5  /* fl(fl(fl(I*c) + corr) * s[0]), per-tensor zero-point */

typedef struct scmp_epilogue {
    int kind;
    float c;                   /* fl(Q*Q / stoc_len) */
    const float *sa, *sb;      /* per-row scales; chunk k at sa + k*sa_chunk_stride */
    int64_t sa_chunk_stride, sb_chunk_stride;
    int64_t sa_batch_stride, sb_batch_stride;
    const float *s;            /* SCALAR: s[0]; HEAD: s[batch] */
    const float *za, *zb;      /* zero points (ZP_ROWCOL: per row; ZP_SCALAR: [0]) */
    const float *suma, *sumb;  /* row sums of q */
    const float *t3;           /* ZP_SCALAR: fp32(D*za*zb) computed in float64, [0] */
    float dfloat;              /* ZP_ROWCOL: D as fp32 */
} scmp_epilogue;

#define SCMP_GEMM_MFMA 0       /* int8 MFMA (v_mfma_i32_32x32x32_i8) */
#define SCMP_GEMM_VALU 1       /* bit-packed AND + v_bcnt (comparison kernel) */
#define SCMP_GEMM_MFMA_FP4 2   /* FP4 (e2m1) MFMA (v_mfma_f32_32x32x64_f8f6f4); lut is the
                                  table of scmp_build_fp4_lut */

typedef struct scmp_gemm_args {
    const uint8_t *ca;         /* A codes (THERMO), rows padded to a multiple of 256 */
    int64_t lda, bsa;          /* bytes per row (multiple of 16), batch stride (bytes) */
    const uint8_t *cb;         /* B codes (Q), rows padded to a multiple of 256 */
    int64_t ldb, bsb;
    int64_t N, M, D, batch;
    int bipolar;
    int JP;                    /* 16, 32, 64, 128 or 256 */
    const int8_t *lut;         /* nclass x 256 x JP */
    const int32_t *d_class;    /* class of each d (NULL: class 0 for every d) */
    int64_t chunk;             /* d per chunk for a chunked ROWCOL epilogue (0: D) */
    scmp_epilogue epi;
    float *y;                  /* fp32 output, row stride ldy, batch stride bsy (elements) */
    int32_t *iout;             /* int32 output for SCMP_EPI_INT */
    int64_t ldy, bsy;
    int impl;                  /* SCMP_GEMM_MFMA, SCMP_GEMM_VALU or SCMP_GEMM_MFMA_FP4 */
    const uint32_t *bitlut;    /* VALU only: nclass x 256 x 2 x (JP/32) bit planes */
    int tile;                  /* MFMA tile preset (0 = default) */
    int nclass;                /* tables in lut; with d_class the FP4 kernel stages them in
                                  LDS when they fit (0: read them from global memory) */
    void *workspace;           /* FP4 only: >= scmp_sc_gemm_workspace_bytes(args) bytes lets
                                  the persistent kernel share tiles between workgroups so
                                  that every CU gets equal work; NULL: whole tiles only */
    int64_t workspace_bytes;
    const int64_t *row_map;    /* output row of A row n (y / iout row row_map[n], each a valid
                                  output row): scatters a row subset in place; NULL: n */
    const int32_t *group_class; /* FP4, not chunked: class of each group of 8 code columns
                                  (D / 8 rounded up entries, D a multiple of 8), every column
                                  of a group in that class; the kernel stages a class table
                                  in LDS where the class changes (codes laid out by class
                                  runs: scmp_permute_code_columns). d_class must be NULL.
                                  NULL: no grouping */
} scmp_gemm_args;

int scmp_sc_gemm(const scmp_gemm_args *args, hipStream_t stream);

/* Workspace the FP4 kernel uses for args (0 when it would not share tiles): per-tile
 * counters and two 256 x 256 slots of exact partial sums per persistent workgroup. The
 * counters are reset by the library on the stream before each launch. No counterpart in
 * the reference (its tiled kernel has one program per output tile,
 * scmp_kernels/sc/kernels.py:838-866). */
int64_t scmp_sc_gemm_workspace_bytes(const scmp_gemm_args *args);

/* scmp_sc_gemm without any allocation: the same kernels and results, with the FP4 kernel's
 * split-tile workspace taken from a static device array of the library
 * (SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES per device, held from the library's first use of
 * the device until the process ends) instead of from the caller. args->workspace must be
 * NULL and args->workspace_bytes 0. A problem whose scmp_sc_gemm_workspace_bytes exceeds
 * the scratch returns SCMP_E_ARG before any device work. The scratch keeps the last
 * call's contents; the library clears what must start at zero (the tile counters, by a
 * kernel on the stream). Every call on one device shares that device's scratch, so calls
 * that overlap on one device (different streams or host threads) race.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
#define SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES ((int64_t)129 << 20)
int scmp_sc_gemm_noalloc(const scmp_gemm_args *args, hipStream_t stream);

/* FP4 (e2m1) form of a stream table for SCMP_GEMM_MFMA_FP4: JPF = max(JP, 32) nibbles per
 * row (JPF / 2 bytes), dword u nibble b holds interval j' = 8u + b (JP = 16: dwords 0 and 1,
 * dwords 2 and 3 zero). Counts that e2m1 cannot represent exactly (anything but 0, 1,
 * 2, 3, 4, 6) set *bad to 1; the table is then unusable and the int8 kernel must be used. */
int scmp_build_fp4_lut(const int8_t *lut, int nclass, int JP, uint8_t *lut4, int32_t *bad,
                       hipStream_t stream);

/* Code columns rearranged into class runs for scmp_gemm_args.group_class: out[r][p] =
 * in[r][src[p]] for src[p] >= 0, 0 for src[p] < 0 (padding of a run to whole groups of 8)
 * and for ncols <= p < ld_out; rows 0..rows-1 of both buffers; every src[p] < ld_in (not
 * checked: src is device memory), ld_out a multiple of 16. No counterpart in the
 * reference (it reads each d's table through the d's class in its tiled kernel,
 * scmp_kernels/sc/kernels.py:176-252). */
int scmp_permute_code_columns(const uint8_t *in, int64_t rows, int64_t ld_in,
                              const int32_t *src, int64_t ncols, uint8_t *out, int64_t ld_out,
                              hipStream_t stream);

/* Bit planes of a stream table for SCMP_GEMM_VALU: bitlut[c][row][plane][w] bit u of
 * word w is bit `plane` of |lut[c][row][j']| for j' = 32w + u (logical interval order). */
int scmp_build_bitlut(const int8_t *lut, int nclass, int JP, uint32_t *bitlut,
                      hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SCMP_HIP_H */
