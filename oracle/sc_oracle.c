/*
 * sc_oracle.c -- CPU restatement of the stochastic-computing (SC) matmul path of
 * swalther06/scmp_kernels, used ONLY as a parity checker.
 *
 * TEST INFRASTRUCTURE. Nothing in the product (scmp_kernels_amd/) links or calls this
 * file. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Every function cites the reference file:line it restates (paths relative to the
 * reference repo root). Floating-point work is IEEE fp32 with one rounding per
 * operation: build with -ffp-contract=off and without fast-math (see Makefile).
 *
 * Parity pins (what each function is checked against) are listed in oracle/README.md
 * and exercised by tests/test_oracle_*.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#pragma STDC FP_CONTRACT OFF

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------------
 * RNG sequences
 * ---------------------------------------------------------------------------------- */

/* Sobol direction vectors, scmp_kernels/sc/rng.py:173-183:
 *   v = int(seed[i] / (1 << (i + 1)) * (1 << length))
 * evaluated in float64 and truncated toward zero like Python's int(). */
EXPORT void orc_sobol_dirvec(int p, const int64_t *seed, int64_t *V) {
    for (int i = 0; i < p; ++i) {
        double v = (double)seed[i] / (double)(1LL << (i + 1)) * (double)(1LL << p);
        V[i] = (int64_t)v;
    }
}

/* Gray-code Sobol stepping, scmp_kernels/sc/rng.py:185-225: return the value before the
 * XOR; index i steps with V[lsz(i)] when lsz(i) < p; lsz(0) = 0. */
EXPORT void orc_sobol(int p, const int64_t *V, int64_t n, int32_t *out) {
    int64_t value = 0;
    for (int64_t idx = 0; idx < n; ++idx) {
        out[idx] = (int32_t)value;
        int k = 0;
        while ((idx >> k) & 1) ++k;          /* least-significant zero of idx */
        if (k < p) value ^= V[k];
    }
}

/* Fibonacci right-shift LFSR, scmp_kernels/sc/rng.py:55-77: output the register, then
 * shift right and insert the XOR of the tapped bits at the top. */
EXPORT void orc_lfsr(int length, int64_t seed, const int32_t *taps, int ntaps, int64_t n,
                     int32_t *out) {
    int64_t reg = seed;
    for (int64_t i = 0; i < n; ++i) {
        out[i] = (int32_t)reg;
        int64_t x = 0;
        for (int t = 0; t < ntaps; ++t) x ^= (reg >> taps[t]) & 1;
        reg = (reg >> 1) | (x << (length - 1));
    }
}

/* Maximal-length check of an LFSR tap set, scmp_kernels/sc/lfsr_taps.py:99-111: step the
 * register from seed 1 for up to period + 1 cycles, recording the values seen; at the first
 * value seen twice return the number of distinct values (the reference compares it with
 * 2^n - 1), else the number recorded. Visited set: a 2^n-bit map (n <= 24). */
EXPORT int64_t orc_lfsr_distinct(int n, const int32_t *taps, int ntaps) {
    const int64_t period = ((int64_t)1 << n) - 1;
    uint8_t *seen = (uint8_t *)calloc((size_t)(((int64_t)1 << n) + 7) / 8, 1);
    int64_t reg = 1, count = 0;
    for (int64_t i = 0; i < period + 1; ++i) {
        const int64_t val = reg;
        int64_t x = 0;
        for (int t = 0; t < ntaps; ++t) x ^= (reg >> taps[t]) & 1;
        reg = (reg >> 1) | (x << (n - 1));
        if (seen[val >> 3] & (1u << (val & 7))) break;
        seen[val >> 3] |= (uint8_t)(1u << (val & 7));
        ++count;
    }
    free(seen);
    return count;
}

/* Bit permutation, scmp_kernels/sc/sng.py:15-29: output bit i = input bit perm[i]. */
EXPORT void orc_scramble(const int32_t *seq, int64_t n, const int32_t *perm, int plen,
                         int32_t *out) {
    for (int64_t t = 0; t < n; ++t) {
        int32_t r = 0;
        for (int i = 0; i < plen; ++i) r |= ((seq[t] >> perm[i]) & 1) << i;
        out[t] = r;
    }
}

/* Prefix / Owen XOR / rescale, scmp_kernels/sc/kernels.py:673-704.
 * r: D x full_len (full_len = 2^p); out: D x L. masks: per-d XOR mask or NULL (mode off).
 * grid = R (rng_levels), base = 2^p. */
EXPORT void orc_prepare_prefix(const int32_t *r, int D, int full_len, int p, int L, int R,
                               const int32_t *masks, int scramble_rescale, int32_t *out) {
    int64_t base = 1LL << p;
    int is_prefix = L < full_len;
    for (int d = 0; d < D; ++d) {
        for (int t = 0; t < L; ++t) {
            int64_t v = r[(int64_t)d * full_len + t];
            if (R == base) {
                if (is_prefix && masks) v ^= masks[d];
            } else {
                if (scramble_rescale && masks) v ^= masks[d];
                int64_t num = v * (int64_t)R;
                /* torch.div(..., rounding_mode="floor") */
                int64_t q = num / base;
                if ((num % base != 0) && ((num < 0) != (base < 0))) q -= 1;
                v = q;
            }
            out[(int64_t)d * L + t] = (int32_t)v;
        }
    }
}

/* bit reverse of the low n bits, scmp_kernels/sc/kernels.py:638-643 */
EXPORT int32_t orc_bitrev(int32_t x, int nbits) {
    int32_t y = 0;
    for (int i = 0; i < nbits; ++i) y |= ((x >> i) & 1) << (nbits - 1 - i);
    return y;
}

/* ------------------------------------------------------------------------------------
 * Enable-signal tables
 * ---------------------------------------------------------------------------------- */

/* K[d,v] = #{t < L : r[d,t] < v}, scmp_kernels/sc/kernels.py:140-169 (v_range > r). */
EXPORT void orc_k_table(const int32_t *r, int D, int L, int V, int16_t *K) {
    for (int d = 0; d < D; ++d)
        for (int v = 0; v < V; ++v) {
            int c = 0;
            for (int t = 0; t < L; ++t) c += (v > r[(int64_t)d * L + t]);
            K[(int64_t)d * V + v] = (int16_t)c;
        }
}

/* C[d,k,v] = #{i < k : r[d,i] < v}, scmp_kernels/sc/kernels.py:102-137. */
EXPORT void orc_c_table(const int32_t *r, int D, int L, int V, int16_t *C) {
    for (int d = 0; d < D; ++d) {
        int16_t *Cd = C + (int64_t)d * (L + 1) * V;
        for (int v = 0; v < V; ++v) Cd[v] = 0;
        for (int k = 0; k < L; ++k) {
            int32_t rv = r[(int64_t)d * L + k];
            for (int v = 0; v < V; ++v)
                Cd[(int64_t)(k + 1) * V + v] = (int16_t)(Cd[(int64_t)k * V + v] + (v > rv));
        }
    }
}

/* ------------------------------------------------------------------------------------
 * Integer accumulator I[n,m] = sum_d s_a s_b C[d, K[d, beta_a], beta_b]
 * (scmp_kernels/sc/kernels.py:216-245; fp32 accumulation of exact integers there).
 * tab_of[d] selects which table row-block (of K and C) serves dimension d, so identical
 * per-d tables may be stored once; pass NULL for tab_of to use d itself.
 * s_a / s_b may be NULL (unipolar: no signs, kernels.py:237-245).
 * ---------------------------------------------------------------------------------- */
EXPORT void orc_sc_accum(const int16_t *beta_a, const int8_t *s_a, const int16_t *beta_b,
                         const int8_t *s_b, int N, int M, int D, const int16_t *K,
                         const int16_t *C, const int32_t *tab_of, int L, int V, int32_t *I,
                         int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int n = 0; n < N; ++n) {
        for (int m = 0; m < M; ++m) {
            int32_t acc = 0;
            const int16_t *ba = beta_a + (int64_t)n * D;
            const int16_t *bb = beta_b + (int64_t)m * D;
            for (int d = 0; d < D; ++d) {
                int td = tab_of ? tab_of[d] : d;
                int k = K[(int64_t)td * V + ba[d]];
                int c = C[((int64_t)td * (L + 1) + k) * V + bb[d]];
                if (s_a) c *= (int)s_a[(int64_t)n * D + d] * (int)s_b[(int64_t)m * D + d];
                acc += c;
            }
            I[(int64_t)n * M + m] = acc;
        }
    }
}

/* Same sum evaluated from the streams themselves (no tables): for each d, count positions
 * t < K[d,beta_a] whose B-side random value is below beta_b. Independent of orc_c_table,
 * used to pin it. */
EXPORT void orc_sc_accum_stream(const int16_t *beta_a, const int8_t *s_a,
                                const int16_t *beta_b, const int8_t *s_b, int N, int M, int D,
                                const int32_t *ra, const int32_t *rb, int L, int32_t *I) {
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) {
            int32_t acc = 0;
            for (int d = 0; d < D; ++d) {
                int va = beta_a[(int64_t)n * D + d], vb = beta_b[(int64_t)m * D + d];
                int k = 0;
                for (int t = 0; t < L; ++t) k += (ra[(int64_t)d * L + t] < va);
                int c = 0;
                for (int t = 0; t < k; ++t) c += (rb[(int64_t)d * L + t] < vb);
                if (s_a) c *= (int)s_a[(int64_t)n * D + d] * (int)s_b[(int64_t)m * D + d];
                acc += c;
            }
            I[(int64_t)n * M + m] = acc;
        }
}

/* ------------------------------------------------------------------------------------
 * Quantizers
 * ---------------------------------------------------------------------------------- */

static inline float rne(float x) { return nearbyintf(x); } /* default mode: half-to-even */
/* std::min / std::max (torch clamp) and numpy minimum / maximum (the Triton interpreter):
 * on ties, including -0.0 vs +0.0, the first argument is returned. */
static inline float fminf_(float a, float b) { return b < a ? b : a; }
static inline float fmaxf_(float a, float b) { return a < b ? b : a; }

/* fused_quant_kernel, PER_ROW + IS_BIPOLAR, scmp_kernels/quant/fused.py:65-81, 98-112:
 *   A = max(max|x|, 1e-5f); scale = A / Q; inv = 1 / scale; q = clamp(rne(x * inv), +-Q)
 *   sign in {-1, 0, +1}; beta = rne(|q| * fl(R / Q)). */
EXPORT void orc_quant_fused_perrow_bipolar(const float *x, int rows, int cols, int Q, int R,
                                           int16_t *beta, int8_t *sign, float *scale) {
    const float eps = 1e-5f, qf = (float)Q, rq = (float)R / (float)Q;
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (int64_t)r * cols;
        float A = 0.0f;
        for (int c = 0; c < cols; ++c) A = fmaxf_(A, fabsf(xr[c]));
        A = fmaxf_(A, eps);
        float s = A / qf;
        float inv = 1.0f / s;
        scale[r] = s;
        for (int c = 0; c < cols; ++c) {
            float v = xr[c] * inv;
            v = rne(v);
            v = fminf_(fmaxf_(v, -qf), qf);
            int64_t o = (int64_t)r * cols + c;
            sign[o] = v > 0.0f ? 1 : (v < 0.0f ? -1 : 0);
            beta[o] = (int16_t)rne(fabsf(v) * rq);
        }
    }
}

/* fused_quant_kernel, flat + IS_BIPOLAR, scmp_kernels/quant/fused.py:86-94, 98-112.
 * inv is the host scale's reciprocal already rounded to fp32 (Triton float argument). */
EXPORT void orc_quant_fused_flat_bipolar(const float *x, int64_t n, float inv, int Q, int R,
                                         int16_t *beta, int8_t *sign) {
    const float qf = (float)Q, rq = (float)R / (float)Q;
    for (int64_t i = 0; i < n; ++i) {
        float v = rne(x[i] * inv);
        v = fminf_(fmaxf_(v, -qf), qf);
        sign[i] = v > 0.0f ? 1 : (v < 0.0f ? -1 : 0);
        beta[i] = (int16_t)rne(fabsf(v) * rq);
    }
}

/* fused_quant_kernel, unipolar (flat or PER_ROW with row_sum),
 * scmp_kernels/quant/fused.py:83-84, 95-96, 113-123: q = clamp(rne(fl(x*inv) + zp), 0, Q);
 * beta = rne(q * fl(R/Q)) (int32); row_sum = sum of q over the row (exact integers). */
EXPORT void orc_quant_fused_unipolar(const float *x, int rows, int cols, float inv, float zp,
                                     int Q, int R, int32_t *beta, float *rowsum) {
    const float qf = (float)Q, rq = (float)R / (float)Q;
    for (int r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (int c = 0; c < cols; ++c) {
            int64_t o = (int64_t)r * cols + c;
            float t = x[o] * inv;
            t = t + zp;
            float v = rne(t);
            v = fminf_(fmaxf_(v, 0.0f), qf);
            sum += v;
            beta[o] = (int32_t)rne(v * rq);
        }
        if (rowsum) rowsum[r] = (float)sum;
    }
}

/* fused_quant_bipolar_batched_kernel, scmp_kernels/quant/fused.py:237-283:
 * q = clamp(rne(x * inv[bh]), -(Q+1), Q); transposed store to (BH, cols, rows). */
EXPORT void orc_quant_batched_bipolar(const float *x, int BH, int rows, int cols,
                                      const float *inv, int Q, int R, int16_t *beta_t,
                                      int8_t *sign_t) {
    const float qmax = (float)Q, qmin = (float)(-(Q + 1)), rq = (float)R / (float)Q;
    for (int b = 0; b < BH; ++b)
        for (int r = 0; r < rows; ++r)
            for (int c = 0; c < cols; ++c) {
                float v = rne(x[((int64_t)b * rows + r) * cols + c] * inv[b]);
                v = fminf_(fmaxf_(v, qmin), qmax);
                int64_t o = ((int64_t)b * cols + c) * rows + r;
                sign_t[o] = v > 0.0f ? 1 : (v < 0.0f ? -1 : 0);
                beta_t[o] = (int16_t)rne(fabsf(v) * rq);
            }
}

/* _grouped_symmetric_quant, scmp_kernels/quant/grouped.py:13-75: groups of G consecutive
 * rows (the remainder rows form the last group); scale = max(max|x|, 1e-5f) / Q;
 * q = clamp(rne(x / scale), +-Q) (division); sign = sgn(q) with 0 -> +1. */
EXPORT void orc_grouped_sym(const float *x, int rows, int cols, int G, int Q,
                            float *scale_row, float *x_int, int8_t *sign) {
    const float eps = 1e-5f, qf = (float)Q;
    if (G >= rows) G = rows;
    for (int g0 = 0; g0 < rows; g0 += G) {
        int g1 = g0 + G < rows ? g0 + G : rows;
        float A = 0.0f;
        for (int r = g0; r < g1; ++r)
            for (int c = 0; c < cols; ++c) A = fmaxf_(A, fabsf(x[(int64_t)r * cols + c]));
        A = fmaxf_(A, eps);
        float s = A / qf;
        for (int r = g0; r < g1; ++r) {
            scale_row[r] = s;
            for (int c = 0; c < cols; ++c) {
                int64_t o = (int64_t)r * cols + c;
                float v = rne(x[o] / s);
                v = fminf_(fmaxf_(v, -qf), qf);
                x_int[o] = v;
                sign[o] = v < 0.0f ? -1 : 1;
            }
        }
    }
}

/* _grouped_asymmetric_quant, scmp_kernels/quant/grouped.py:78-133:
 * range = max(mx - mn, 1e-5f); scale = range / Q; zp = clamp(rne(-mn / scale), 0, Q);
 * q = clamp(rne(fl(x / scale) + zp), 0, Q). */
EXPORT void orc_grouped_asym(const float *x, int rows, int cols, int G, int Q,
                             float *scale_row, float *zp_row, float *x_int) {
    const float eps = 1e-5f, qf = (float)Q;
    if (G >= rows) G = rows;
    for (int g0 = 0; g0 < rows; g0 += G) {
        int g1 = g0 + G < rows ? g0 + G : rows;
        float mx = -INFINITY, mn = INFINITY;
        for (int r = g0; r < g1; ++r)
            for (int c = 0; c < cols; ++c) {
                float v = x[(int64_t)r * cols + c];
                mx = fmaxf_(mx, v);
                mn = fminf_(mn, v);
            }
        float range = mx - mn;
        range = fmaxf_(range, eps);
        float s = range / qf;
        float nmn = -mn;
        float zp = rne(nmn / s);
        zp = fminf_(fmaxf_(zp, 0.0f), qf);
        for (int r = g0; r < g1; ++r) {
            scale_row[r] = s;
            zp_row[r] = zp;
            for (int c = 0; c < cols; ++c) {
                int64_t o = (int64_t)r * cols + c;
                float t = x[o] / s;
                t = t + zp;
                float v = rne(t);
                x_int[o] = fminf_(fmaxf_(v, 0.0f), qf);
            }
        }
    }
}

/* Boundary remap of the grouped paths, scmp_kernels/sc/kernels.py:1679-1686:
 * beta = rne(fl(fl(|q| * R) / Q)) (abs only for bipolar). */
EXPORT void orc_beta_from_q_div(const float *q, int64_t n, int Q, int R, int absval,
                                int16_t *beta) {
    const float qf = (float)Q, rf = (float)R;
    for (int64_t i = 0; i < n; ++i) {
        float v = absval ? fabsf(q[i]) : q[i];
        float t = v * rf;
        t = t / qf;
        beta[i] = (int16_t)rne(t);
    }
}

/* Boundary remap of the batched 3D grouped path, scmp_kernels/sc/kernels.py:1864-1865:
 * beta = rne(|q| * fp32(R / Q)) with R / Q evaluated in float64 then cast. */
EXPORT void orc_beta_from_q_mul(const float *q, int64_t n, int Q, int R, int16_t *beta) {
    const float rq = (float)((double)R / (double)Q);
    for (int64_t i = 0; i < n; ++i) beta[i] = (int16_t)rne(fabsf(q[i]) * rq);
}
