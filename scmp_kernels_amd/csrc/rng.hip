// RNG sequence generation, Owen scramble / rescale and the stream tables of the SC GEMM.
//
// Sequences are tiny (D x 2^p int32, p <= 8 here) and built once per configuration and
// cached by the host; these kernels are about getting the integers right, not speed.
#include <stdarg.h>

#include "common.h"

namespace scmp {

static thread_local char g_err[512];

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

struct SobolV {
    int64_t v[32];
};

// x_t = XOR of V_k over the set bits k < p of gray(t) = t ^ (t >> 1): the closed form of
// the return-before-XOR Gray-code stepping of scmp_kernels/sc/rng.py:199-206 (valid for
// t < 2^p, the only lengths requested: sequences are 2^sc_prec long, kernels.py:78-85).
__global__ void sobol_kernel(int p, SobolV V, int64_t n, int32_t *out) {
    int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= n) return;
    uint64_t g = (uint64_t)t ^ ((uint64_t)t >> 1);
    int64_t x = 0;
    for (int k = 0; k < p; ++k)
        if ((g >> k) & 1) x ^= V.v[k];
    out[t] = (int32_t)x;
}

// Sequential stepping (one thread): used when n exceeds the closed form's range.
__global__ void sobol_serial_kernel(int p, SobolV V, int64_t n, int32_t *out) {
    int64_t value = 0;
    for (int64_t i = 0; i < n; ++i) {
        out[i] = (int32_t)value;
        int k = __builtin_ctzll(~(uint64_t)i);
        if (k < p) value ^= V.v[k];
    }
}

// LFSR state is sequential; one thread steps it (n <= 2^16 here).
__global__ void lfsr_kernel(int length, int64_t seed, uint64_t taps, int64_t n, int32_t *out) {
    uint64_t reg = (uint64_t)seed;
    for (int64_t i = 0; i < n; ++i) {
        out[i] = (int32_t)reg;
        uint64_t x = __builtin_popcountll(reg & taps) & 1;
        reg = (reg >> 1) | (x << (length - 1));
    }
}

// Maximal-length test of Fibonacci LFSR tap sets, one candidate per thread. The state
// sequence from seed 1 (s_{k+1} = (s_k >> 1) | (parity(s_k & mask) << (n - 1))) is
// eventually periodic; Brent's cycle detection finds its period lam and pre-period mu with
// O(mu + lam) steps and O(1) state. mu + lam is the number of distinct states before the
// first repeat; _is_maximal_length (scmp_kernels/sc/lfsr_taps.py:99-111) accepts a tap set
// when that number equals the expected period 2^n - 1. Every loop is bounded by the 2^n
// states of the register.
__device__ __forceinline__ uint32_t lfsr_next(uint32_t x, uint32_t mask, int n) {
    return (x >> 1) | ((uint32_t)(__builtin_popcount(x & mask) & 1) << (n - 1));
}

__global__ void lfsr_distinct_kernel(int n, const uint32_t *masks, int64_t count,
                                     uint32_t *distinct) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint32_t mask = masks[i];
    const uint32_t x0 = 1u;
    // Brent: lam = period
    uint32_t power = 1, lam = 1;
    uint32_t tort = x0, hare = lfsr_next(x0, mask, n);
    while (tort != hare) {
        if (power == lam) {
            tort = hare;
            power <<= 1;
            lam = 0;
        }
        hare = lfsr_next(hare, mask, n);
        ++lam;
    }
    // mu = first index of the cycle: advance one pointer lam steps, then both together
    tort = hare = x0;
    for (uint32_t k = 0; k < lam; ++k) hare = lfsr_next(hare, mask, n);
    uint32_t mu = 0;
    while (tort != hare) {
        tort = lfsr_next(tort, mask, n);
        hare = lfsr_next(hare, mask, n);
        ++mu;
    }
    distinct[i] = mu + lam;
}

__global__ void expand_kernel(const int32_t *base, int64_t n, const int32_t *src,
                              const int32_t *perm, int p, int D, int32_t *out) {
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)D * n) return;
    int d = (int)(i / n);
    int64_t t = i - (int64_t)d * n;
    int32_t v = base[(int64_t)src[d] * n + t];
    if (perm && perm[(int64_t)d * p] >= 0) {
        const int32_t *pp = perm + (int64_t)d * p;
        int32_t r = 0;
        for (int b = 0; b < p; ++b) r |= ((v >> pp[b]) & 1) << b;
        v = r;
    }
    out[i] = v;
}

__global__ void prepare_kernel(const int32_t *r, int D, int full, int p, int L, int R,
                               const int32_t *masks, int scramble_rescale, int32_t *out) {
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= (int64_t)D * L) return;
    int d = (int)(i / L), t = (int)(i - (int64_t)d * L);
    int64_t base = 1LL << p;
    int64_t v = r[(int64_t)d * full + t];
    if (R == base) {
        if (L < full && masks) v ^= masks[d];
    } else {
        if (scramble_rescale && masks) v ^= masks[d];
        int64_t num = v * (int64_t)R;
        int64_t q = num / base;                       // floor division (torch "floor")
        if ((num % base != 0) && (num < 0)) q -= 1;
        v = q;
    }
    out[i] = (int32_t)v;
}

// Boundary of magnitude q on the RNG grid: rne(fl(fl(q*R)/Q)). The fused form
// rne(q * fl(R/Q)) gives the same integer for odd Q and power-of-two R (q*R/Q is never
// a half-integer and the two fp32 values differ by at most 1 ulp of a value <= 2R).
__device__ __forceinline__ int beta_of(int q, int Q, int R) {
    float t = __fmul_rn((float)q, (float)R);
    t = __fdiv_rn(t, (float)Q);
    return (int)rne(t);
}

// One block per class. Threads cooperate on the count tables; thread 0 derives the
// interval boundaries kappa (a short sequential scan over q).
__global__ void stream_tables_kernel(const int32_t *ra_all, const int32_t *rb_all,
                                     const int32_t *rep, int L, int p, int R, int bipolar,
                                     int JP, uint8_t *jtab, int8_t *lut, int16_t *kappa,
                                     int32_t *jmax_out) {
    extern __shared__ int32_t sm[];
    int c = blockIdx.x;
    int d = rep[c];
    const int32_t *ra = ra_all + (int64_t)d * L;
    const int32_t *rb = rb_all + (int64_t)d * L;
    int Q = bipolar ? (1 << (p - 1)) - 1 : (1 << p) - 1;
    int qmax = bipolar ? Q + 1 : Q;                   // per-head clamp admits |q| = Q+1
    // sm layout: K of each q (qmax+1), kappa (JP+1), j of each q (256), rb (L)
    int32_t *Kq = sm;
    int32_t *kap = Kq + 257;
    int32_t *jq = kap + 257;
    int32_t *rbs = jq + 256;
    for (int t = threadIdx.x; t < L; t += blockDim.x) rbs[t] = rb[t];
    for (int q = threadIdx.x; q <= qmax; q += blockDim.x) {
        int v = beta_of(q, Q, R);
        int k = 0;
        for (int t = 0; t < L; ++t) k += (ra[t] < v);
        Kq[q] = k;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int J = 0;
        kap[0] = 0;
        for (int q = 0; q <= qmax; ++q) {
            int k = Kq[q];
            if (k > kap[J]) {
                ++J;
                if (J <= JP) kap[J] = k;
            }
            jq[q] = J;
        }
        for (int q = qmax + 1; q < 256; ++q) jq[q] = J;
        atomicMax(jmax_out, J);
        if (J > JP) J = JP;                            // reported through jmax_out
        for (int j = J + 1; j <= JP; ++j) kap[j] = kap[J];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < 256; q += blockDim.x) jtab[(int64_t)c * 256 + q] = (uint8_t)jq[q];
    for (int j = threadIdx.x; j <= JP; j += blockDim.x) kappa[(int64_t)c * (JP + 1) + j] = (int16_t)kap[j];
    // lut rows: row = code byte; q = (int8)row (bipolar) or row (unipolar)
    int8_t *lc = lut + (int64_t)c * 256 * JP;
    int U = JP / 4;
    for (int e = threadIdx.x; e < 256 * JP; e += blockDim.x) {
        int row = e / JP, byte = e - row * JP;
        int u = byte >> 2, b = byte & 3;
        int jp = U * b + u;
        int q = bipolar ? (int)(int8_t)(uint8_t)row : row;
        int s = q < 0 ? -1 : 1;
        int mag = q < 0 ? -q : q;
        int val = 0;
        if (mag <= qmax && jp < JP) {
            int v = beta_of(mag, Q, R);
            int i0 = kap[jp], i1 = kap[jp + 1];
            for (int i = i0; i < i1; ++i) val += (rbs[i] < v);
        }
        lc[e] = (int8_t)(s * val);
    }
}

__global__ void bitlut_kernel(const int8_t *lut, int nclass, int JP, uint32_t *bitlut) {
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int W = JP / 32 > 0 ? JP / 32 : 1;
    int64_t total = (int64_t)nclass * 256 * 2 * W;
    if (i >= total) return;
    int w = (int)(i % W);
    int plane = (int)((i / W) % 2);
    int64_t cr = i / (2 * W);                          // class * 256 + row
    const int8_t *row = lut + cr * JP;
    int U = JP / 4;
    uint32_t bits = 0;
    for (int u = 0; u < 32; ++u) {
        int jp = 32 * w + u;
        if (jp >= JP) break;
        int byte = 4 * (jp % U) + jp / U;              // inverse of jp = U*b + u'
        int v = row[byte];
        v = v < 0 ? -v : v;
        bits |= (uint32_t)((v >> plane) & 1) << u;
    }
    bitlut[i] = bits;
}

}  // namespace scmp

using namespace scmp;

extern "C" {

int scmp_abi_version(void) { return 3; }

const char *scmp_last_error(void) { return g_err; }

int scmp_rng_sobol(int p, const int64_t *V_host, int64_t n, int32_t *out, hipStream_t stream) {
    SCMP_REQUIRE(p >= 1 && p <= 30, "scmp_rng_sobol: p=%d out of range [1, 30]", p);
    SCMP_REQUIRE(n >= 0 && out, "scmp_rng_sobol: bad n/out");
    if (n == 0) return SCMP_OK;
    SobolV V;
    for (int k = 0; k < p; ++k) V.v[k] = V_host[k];
    if (n <= (1LL << p)) {
        sobol_kernel<<<cdiv(n, 256), 256, 0, stream>>>(p, V, n, out);
    } else {
        sobol_serial_kernel<<<1, 1, 0, stream>>>(p, V, n, out);
    }
    SCMP_LAUNCH_CHECK("scmp_rng_sobol");
    return SCMP_OK;
}

int scmp_rng_lfsr(int length, int64_t seed, uint64_t taps_mask, int64_t n, int32_t *out,
                  hipStream_t stream) {
    SCMP_REQUIRE(length >= 1 && length <= 62, "scmp_rng_lfsr: length=%d out of range", length);
    SCMP_REQUIRE(seed != 0, "LFSR seed must be non-zero");
    SCMP_REQUIRE(n >= 0 && out, "scmp_rng_lfsr: bad n/out");
    if (n == 0) return SCMP_OK;
    lfsr_kernel<<<1, 1, 0, stream>>>(length, seed, taps_mask, n, out);
    SCMP_LAUNCH_CHECK("scmp_rng_lfsr");
    return SCMP_OK;
}

int scmp_lfsr_search(int n_bits, const uint32_t *masks, int64_t count, uint32_t *distinct,
                     hipStream_t stream) {
    SCMP_REQUIRE(n_bits >= 2 && n_bits <= SCMP_LFSR_SEARCH_MAX_BITS,
                 "scmp_lfsr_search: n_bits=%d out of range [2, %d]", n_bits,
                 SCMP_LFSR_SEARCH_MAX_BITS);
    SCMP_REQUIRE(masks && distinct && count >= 0, "scmp_lfsr_search: bad arguments");
    if (count == 0) return SCMP_OK;
    lfsr_distinct_kernel<<<cdiv(count, 256), 256, 0, stream>>>(n_bits, masks, count,
                                                               distinct);
    SCMP_LAUNCH_CHECK("scmp_lfsr_search");
    return SCMP_OK;
}

int scmp_rng_expand(const int32_t *base, int64_t n, const int32_t *src, const int32_t *perm,
                    int p, int D, int32_t *out, hipStream_t stream) {
    SCMP_REQUIRE(base && src && out && n > 0 && D > 0 && p >= 1 && p <= 31,
                 "scmp_rng_expand: bad arguments (n=%lld D=%d p=%d)", (long long)n, D, p);
    int64_t total = (int64_t)D * n;
    expand_kernel<<<cdiv(total, 256), 256, 0, stream>>>(base, n, src, perm, p, D, out);
    SCMP_LAUNCH_CHECK("scmp_rng_expand");
    return SCMP_OK;
}

int scmp_rng_prepare(const int32_t *r, int D, int full, int p, int L, int R,
                     const int32_t *masks, int scramble_rescale, int32_t *out,
                     hipStream_t stream) {
    SCMP_REQUIRE(r && out && D > 0 && full > 0 && L > 0 && L <= full && R > 0,
                 "scmp_rng_prepare: bad arguments (D=%d full=%d L=%d R=%d)", D, full, L, R);
    SCMP_REQUIRE(p >= 1 && p <= 30, "scmp_rng_prepare: p=%d out of range", p);
    int64_t total = (int64_t)D * L;
    prepare_kernel<<<cdiv(total, 256), 256, 0, stream>>>(r, D, full, p, L, R, masks,
                                                        scramble_rescale, out);
    SCMP_LAUNCH_CHECK("scmp_rng_prepare");
    return SCMP_OK;
}

int scmp_build_stream_tables(const int32_t *ra, const int32_t *rb, const int32_t *rep,
                             int nclass, int L, int p, int R, int bipolar, int JP,
                             uint8_t *jtab, int8_t *lut, int16_t *kappa, int32_t *jmax_out,
                             hipStream_t stream) {
    SCMP_REQUIRE(ra && rb && rep && jtab && lut && kappa && jmax_out && nclass > 0,
                 "scmp_build_stream_tables: null argument");
    SCMP_REQUIRE(p >= 1 && p <= 8, "scmp_build_stream_tables: sc_prec=%d unsupported "
                 "(8-bit codes need sc_prec <= 8)", p);
    SCMP_REQUIRE(JP == 16 || JP == 32 || JP == 64 || JP == 128 || JP == 256,
                 "scmp_build_stream_tables: JP=%d must be 16, 32, 64, 128 or 256", JP);
    SCMP_REQUIRE(L >= 1 && L <= 4096 && R >= 1, "scmp_build_stream_tables: L=%d R=%d", L, R);
    size_t smem = (257 + 257 + 256 + (size_t)L) * sizeof(int32_t);
    stream_tables_kernel<<<nclass, 256, smem, stream>>>(ra, rb, rep, L, p, R, bipolar, JP,
                                                        jtab, lut, kappa, jmax_out);
    SCMP_LAUNCH_CHECK("scmp_build_stream_tables");
    return SCMP_OK;
}

int scmp_build_bitlut(const int8_t *lut, int nclass, int JP, uint32_t *bitlut,
                      hipStream_t stream) {
    SCMP_REQUIRE(lut && bitlut && nclass > 0 && JP >= 16, "scmp_build_bitlut: bad arguments");
    int W = JP / 32 > 0 ? JP / 32 : 1;
    int64_t total = (int64_t)nclass * 256 * 2 * W;
    bitlut_kernel<<<cdiv(total, 256), 256, 0, stream>>>(lut, nclass, JP, bitlut);
    SCMP_LAUNCH_CHECK("scmp_build_bitlut");
    return SCMP_OK;
}

}  // extern "C"
