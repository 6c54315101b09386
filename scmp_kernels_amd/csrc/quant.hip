// FP -> SC-code quantizers for gfx950.
//
// One pipeline covers the six quantizer variants of the reference (fused per-row /
// per-tensor / per-head Triton kernels and the torch row-group quantizers):
//   1. reduce   : one wavefront per (row, column segment) reduces max|x| or (min, max)
//                 and folds it into its (row group, segment) statistic with an atomic max
//                 on an order-preserving integer key (max/min are exact, so the result is
//                 independent of reduction order);
//   2. finalize : one thread per (group, segment) derives scale / reciprocal / zero-point
//                 with the variant's fp32 (or float64 host-style) operation order;
//   3. quantize : one wavefront per row writes the GEMM code bytes (zero-padded to the
//                 GEMM's row/column padding), the reference API outputs and row sums.
// All three are HBM-bound streaming passes (the second input read mostly hits L2/MALL).
#include "common.h"

namespace scmp {

struct QParams {
    float s, inv, zp, pad;
    double s64, zp64;
};

__device__ __forceinline__ uint32_t key_of(float f) {
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float float_of_key(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

// First element of quantized row r: the caller's row index picks the input row.
__device__ __forceinline__ const float *x_row(const scmp_quant_args &a, int64_t r) {
    return a.x + (a.row_index ? a.row_index[r] : r) * a.ld;
}

// Element c of a row whose start (x_row) the caller has looked up once.
__device__ __forceinline__ float load_x(const scmp_quant_args &a, const float *row, int64_t c) {
    float v = row[c];
    if (a.smooth_mode == SCMP_SMOOTH_DIV) v = __fdiv_rn(v, a.smooth[c]);
    else if (a.smooth_mode == SCMP_SMOOTH_MUL) v = __fmul_rn(v, a.smooth[c]);
    return v;
}

__device__ __host__ __forceinline__ bool is_asym(int variant) {
    return variant == SCMP_Q_GROUP_ASYM || variant == SCMP_Q_TENSOR_ASYM ||
           variant == SCMP_Q_HOST_ASYM;
}

__global__ void stats_init_kernel(uint32_t *stats, int64_t n) {
    int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) stats[i] = 0u;
}

// stats of each (row group) from the caller's max|x| (symmetric variants, one segment)
__global__ void stats_given_kernel(uint32_t *stats, const float *given, int64_t nunits) {
    int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (u >= nunits) return;
    stats[u * 2 + 0] = __float_as_uint(fabsf(given[u]));
    stats[u * 2 + 1] = 0u;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
// Sum over the wave; exact for the integer-valued code sums it is used on (below 2^24).
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// stats[unit*2 + 0] = key(max) or bits(max|x|); stats[unit*2 + 1] = key(-min)
__global__ void reduce_kernel(scmp_quant_args a, int64_t group, int64_t segw, int64_t nseg,
                              uint32_t *stats) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    const int64_t ntask = a.rows * nseg;
    const bool asym = is_asym(a.variant);
    for (int64_t task = wave; task < ntask; task += nwaves) {
        int64_t r = task / nseg, sgi = task - r * nseg;
        int64_t c0 = sgi * segw, c1 = c0 + segw < a.cols ? c0 + segw : a.cols;
        float mx = -INFINITY, mn = INFINITY, am = 0.0f;
        const float *xr = x_row(a, r);
        for (int64_t c = c0 + lane; c < c1; c += 64) {
            float v = load_x(a, xr, c);
            if (asym) {
                mx = fmaxf(mx, v);
                mn = fminf(mn, v);
            } else {
                am = fmaxf(am, fabsf(v));
            }
        }
        int64_t unit = (r / group) * nseg + sgi;
        if (asym) {
            mx = wave_max(mx);
            mn = wave_min(mn);
            if (lane == 0) {
                atomicMax(&stats[unit * 2 + 0], key_of(mx));
                atomicMax(&stats[unit * 2 + 1], key_of(-mn));
            }
        } else {
            am = wave_max(am);
            if (lane == 0) atomicMax(&stats[unit * 2 + 0], __float_as_uint(am));
        }
    }
}

// Scale / reciprocal / zero-point of one (group, segment) from its reduced statistics
// (stat0 = bits of max|x| or key(max), stat1 = key(-min)), in the operation order of the
// variant's reference.
__device__ QParams derive_params(const scmp_quant_args &a, uint32_t stat0, uint32_t stat1) {
    const float eps = 1e-5f;
    const float qf = (float)a.q_max;
    QParams p = {0.f, 0.f, 0.f, 0.f, 0.0, 0.0};
    switch (a.variant) {
    case SCMP_Q_GROUP_SYM:
    case SCMP_Q_ROW_SYM:
    case SCMP_Q_HEAD_SYM: {
        // max(|x|) clamped at 1e-5f; scale = A / Q; inv = 1 / scale (fused kernels,
        // quant/fused.py:76-79; per-head host math kernels.py:490-495; grouped
        // quant/grouped.py:46-47)
        float A = fmax_first(__uint_as_float(stat0), eps);
        p.s = __fdiv_rn(A, qf);
        p.inv = __fdiv_rn(1.0f, p.s);
        p.s64 = (double)p.s;
        break;
    }
    case SCMP_Q_TENSOR_SYM: {
        // Python floats: max(|max|, |min|, 1e-5) / q_max; 1.0 / scale -> fp32 kernel arg
        // (sc/kernels.py:1173-1174, quant/fused.py:172-174)
        double A = (double)__uint_as_float(stat0);
        A = A > 1e-5 ? A : 1e-5;
        p.s64 = __ddiv_rn(A, (double)a.q_max);
        p.inv = (float)__ddiv_rn(1.0, p.s64);
        p.s = (float)p.s64;
        break;
    }
    case SCMP_Q_GROUP_ASYM: {
        // quant/grouped.py:111-115
        float mx = float_of_key(stat0);
        float mn = -float_of_key(stat1);
        float range = fmax_first(__fsub_rn(mx, mn), eps);
        p.s = __fdiv_rn(range, qf);
        float z = rne(__fdiv_rn(-mn, p.s));
        p.zp = fmin_first(fmax_first(z, 0.0f), qf);
        p.inv = __fdiv_rn(1.0f, p.s);
        p.s64 = (double)p.s;
        p.zp64 = (double)p.zp;
        break;
    }
    case SCMP_Q_HOST_SYM:
    case SCMP_Q_HOST_ASYM:
        // the caller computed scale / reciprocal / zero-point in Python floats
        // (quant/fused.py:172-174, 204-209) and passes them rounded to fp32
        p.inv = a.host_inv;
        p.zp = a.host_zp;
        break;
    case SCMP_Q_TENSOR_ASYM: {
        // quant/fused.py:204-209 in Python floats
        double mx = (double)float_of_key(stat0);
        double mn = -(double)float_of_key(stat1);
        double range = mx - mn;
        range = range > 1e-5 ? range : 1e-5;
        p.s64 = __ddiv_rn(range, (double)a.q_max);
        p.inv = (float)__ddiv_rn(1.0, p.s64);
        double z = __builtin_rint(__ddiv_rn(-mn, p.s64));
        z = z < 0.0 ? 0.0 : (z > (double)a.q_max ? (double)a.q_max : z);
        p.zp64 = z;
        p.zp = (float)z;
        p.s = (float)p.s64;
        break;
    }
    }
    return p;
}

__global__ void finalize_kernel(scmp_quant_args a, int64_t nunits, const uint32_t *stats,
                                QParams *prm) {
    int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (u >= nunits) return;
    prm[u] = derive_params(a, stats[u * 2], stats[u * 2 + 1]);
}

// The quantized integer of one element (pre-clamp value t, clamp to [qlo, Q]) in the
// variant's operation order: division by the scale for the torch row-group quantizers,
// multiplication by the reciprocal for the fused Triton ones.
__device__ __forceinline__ float quant_value(const scmp_quant_args &a, const QParams &p,
                                             float v, float qlo, float qf) {
    float t;
    switch (a.variant) {
    case SCMP_Q_GROUP_SYM: t = __fdiv_rn(v, p.s); break;
    case SCMP_Q_GROUP_ASYM: t = __fadd_rn(__fdiv_rn(v, p.s), p.zp); break;
    case SCMP_Q_TENSOR_ASYM:
    case SCMP_Q_HOST_ASYM: t = __fadd_rn(__fmul_rn(v, p.inv), p.zp); break;
    default: t = __fmul_rn(v, p.inv); break;
    }
    return fmin_first(fmax_first(rne(t), qlo), qf);
}

// Writes the optional reference outputs of element (r, c) and returns its GEMM code byte.
__device__ __forceinline__ uint8_t element_outputs(const scmp_quant_args &a, float q,
                                                   int64_t r, int64_t c, bool asym, float rq,
                                                   float rf, float qf) {
    const int64_t o = r * a.out_ld + c;
    if (a.beta16 || a.beta32) {
        const float mag = fabsf(q);
        const float bf = a.beta_formula == 0 ? __fmul_rn(mag, rq)
                                             : __fdiv_rn(__fmul_rn(mag, rf), qf);
        const int bv = (int)rne(bf);
        if (a.beta16) a.beta16[o] = (int16_t)bv;
        if (a.beta32) a.beta32[o] = bv;
    }
    if (a.sign) {
        int8_t sg;
        if (a.variant == SCMP_Q_GROUP_SYM) sg = q < 0.0f ? -1 : 1;
        else sg = q > 0.0f ? 1 : (q < 0.0f ? -1 : 0);
        a.sign[o] = sg;
    }
    if (a.xint) a.xint[o] = q;
    if (!a.code) return 0;
    const int qi = (int)q;
    if (a.code_kind == SCMP_CODE_Q) return (uint8_t)(qi & 0xff);
    const int cls = a.col_class ? a.col_class[c] : 0;
    const int mi = qi < 0 ? -qi : qi;
    uint8_t code = a.jtab[(int64_t)cls * 256 + mi];
    if (!asym && qi < 0) code |= 0x80;
    return code;
}

__global__ void quantize_kernel(scmp_quant_args a, int64_t group, int64_t segw, int64_t nseg,
                                const QParams *prm) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    // rows visited: every code row when codes are written (padding rows get zeros),
    // otherwise every input row
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    const int64_t nbatch = a.code ? a.rows / cbr : 1;
    const int64_t nrows_total = a.code ? nbatch * a.code_rows : a.rows;
    const float qf = (float)a.q_max;
    const bool asym = is_asym(a.variant);
    const float qlo = asym ? 0.0f : (a.variant == SCMP_Q_HEAD_SYM ? -(qf + 1.0f) : -qf);
    const float rq = __fdiv_rn((float)a.rng_levels, qf);
    const float rf = (float)a.rng_levels;
    for (int64_t vr = wave; vr < nrows_total; vr += nwaves) {
        int64_t r = vr, crow = vr;
        if (a.code) {
            const int64_t b = vr / a.code_rows, i = vr - b * a.code_rows;
            if (i >= cbr) {                      // zero code rows of the GEMM padding
                for (int64_t c = lane; c < a.code_ld; c += 64) a.code[vr * a.code_ld + c] = 0;
                continue;
            }
            r = b * cbr + i;
        }
        const int64_t g = r / group;
        float rsum = 0.0f;
        const float *xr = x_row(a, r);
        for (int64_t c = lane; c < a.cols; c += 64) {
            const int64_t sgi = c / segw;
            const QParams p = prm[g * nseg + sgi];
            const float q = quant_value(a, p, load_x(a, xr, c), qlo, qf);
            const uint8_t code = element_outputs(a, q, r, c, asym, rq, rf, qf);
            if (a.code) a.code[crow * a.code_ld + c] = code;
            rsum += q;                            // exact: integers below 2^24
        }
        if (a.code)
            for (int64_t c = a.cols + lane; c < a.code_ld; c += 64) a.code[crow * a.code_ld + c] = 0;
        if (a.rowsum) {
            for (int o = 32; o > 0; o >>= 1) rsum += __shfl_xor(rsum, o, 64);
            if (lane == 0) a.rowsum[r] = rsum;
        }
        if (lane < nseg && (a.scale || a.inv)) {
            for (int64_t sgi = lane; sgi < nseg; sgi += 64) {
                const QParams p = prm[g * nseg + sgi];
                if (a.scale) a.scale[sgi * a.rows + r] = p.s;
                if (a.inv) a.inv[sgi * a.rows + r] = p.inv;
            }
        }
        if (lane == 0 && a.zp) a.zp[r] = prm[g * nseg].zp;
    }
}

// ---------------------------------------------------------------------------------
// One-pass quantizer for row groups (variants GROUP_SYM, GROUP_ASYM, ROW_SYM, HEAD_SYM
// without column segments): one 256-thread workgroup per group of G rows reads the group
// once, reduces its statistic, derives the scale and writes codes and outputs. Elements
// go in chunks of 4 consecutive columns of a row; up to kMaxChunks chunks per thread stay
// in registers between the passes, larger groups re-read their chunks (from L2).
// The reduction performs the same max/min operations as reduce_kernel, so the statistic,
// and everything derived from it, is bit-identical to the three-kernel pipeline.
// The element operation (OP) and the smoothing mode (SM) are template parameters, so the
// per-element path is straight-line code; chunk positions are tracked in 32-bit ints.
// ---------------------------------------------------------------------------------

constexpr int kGroupThreads = 256;
constexpr int kGroupMaxRows = 1024;       // row sums of a group live in LDS
constexpr int kMaxChunks = 16;            // register-held 4-column chunks per thread, max
constexpr int kBigGroupThreads = 1024;    // threads of a workgroup for groups past 256 x 16
constexpr int kMidGroupThreads = 512;     // wide groups when 1024 threads would need 2 rounds
constexpr int kBigChunks = 12;            // register-held chunks per thread at 1024 threads
                                          // (128 registers: 16 would spill)
constexpr int kMidChunks = 20;            // at 512 threads, two workgroups per compute unit

enum { QOP_DIV = 0, QOP_DIVZP = 1, QOP_MUL = 2 };

// rne(fl(x / s)) (OP DIV) or rne(fl(fl(x / s) + zp)) (OP DIVZP), exactly, without the IEEE
// division in the common case. y = fl(x * fl(1/s)) is within |x/s| * 1.2e-7 of x/s; for
// |y| < 1024 that is < 1.3e-4, and the roundings of fl(x/s) and of the zero-point sum add
// < 1.6e-4 more. So when y (or fl(y + zp)) lies farther than 2^-11 from every
// half-integer, the exact value lies strictly on the same side of the same half-integer
// and rounds to the same integer; otherwise (and for |y| >= 1024, inf, NaN) the exact
// division decides.
template <int OP>
__device__ __forceinline__ float rne_quotient(float x, float s, float inv, float zp) {
    const float y = __fmul_rn(x, inv);
    if (__builtin_fabsf(y) < 1024.0f) {
        const float u = OP == QOP_DIVZP ? __fadd_rn(y, zp) : y;
        const float k = rne(u);
        if (__builtin_fabsf(__fsub_rn(u, k)) < 0.5f - 4.8828125e-4f) return k;
    }
    const float t = __fdiv_rn(x, s);
    return rne(OP == QOP_DIVZP ? __fadd_rn(t, zp) : t);
}

// four consecutive floats at a 4-byte aligned address (rows whose stride is not a multiple
// of 4 floats): still one 16-byte load
struct __attribute__((aligned(4))) float4u {
    float x, y, z, w;
};

// Chunk loads that never sit under a branch: a load inside a divergent branch (or one whose
// address comes from an earlier load) makes the compiler wait for every load in flight at
// the branch's end, which serializes a thread's chunks into one memory round trip each.
// So a thread first issues the raw loads of all its chunks, with the chunk start clamped
// into the row, and only then shifts, smooths and uses them.
// MODE 0: rows 16-byte aligned and cols % 4 == 0 (one 16-byte load per chunk, no clamping);
// MODE 1: cols >= 4, any row stride (four 4-byte loads at min(c, cols - 4));
// MODE 2: cols < 4 (four loads at min(c + k, cols - 1)).
template <int MODE>
__device__ __forceinline__ void load_raw4(const float *row, int c, int cols, float (&t)[4]) {
    if constexpr (MODE == 0) {
        const float4 x4 = *(const float4 *)(row + c);
        t[0] = x4.x; t[1] = x4.y; t[2] = x4.z; t[3] = x4.w;
    } else if constexpr (MODE == 1) {
        const int c0 = c < cols - 4 ? c : cols - 4;
        const float4u u = *(const float4u *)(row + c0);
        t[0] = u.x; t[1] = u.y; t[2] = u.z; t[3] = u.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] = row[c + k < cols ? c + k : cols - 1];
    }
}

// Smoothing in the quantizer's fp32 order (x / s or x * s), then the chunk moved to start at
// column c (MODE 1 loads a chunk that runs past the row end from cols - 4) and columns past
// the row end set to 0.
template <int MODE, int SM>
__device__ __forceinline__ void finish4(int c, int cols, float (&t)[4], const float (&sv)[4]) {
    if constexpr (SM != SCMP_SMOOTH_NONE) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            t[k] = SM == SCMP_SMOOTH_DIV ? __fdiv_rn(t[k], sv[k]) : __fmul_rn(t[k], sv[k]);
    }
    if constexpr (MODE == 1) {
        const int sh = c - (c < cols - 4 ? c : cols - 4);      // 0 except at a row end
        if (sh != 0) {
            float u[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) u[k] = t[k];
#pragma unroll
            for (int k = 0; k < 4; ++k) t[k] = k + sh < 4 ? u[k + sh < 4 ? k + sh : 3] : 0.0f;
        }
    } else if constexpr (MODE == 2) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (c + k >= cols) t[k] = 0.0f;
    }
}

// MODE of a quantizer call: 0 when every row start is 16-byte aligned and rows are whole
// chunks, else 1 (2 for rows of fewer than 4 columns).
__device__ __host__ __forceinline__ int chunk_mode(const scmp_quant_args &a) {
    const bool aligned = (a.ld % 4 == 0) && (((uintptr_t)a.x & 15) == 0) &&
                         (a.smooth == nullptr || ((uintptr_t)a.smooth & 15) == 0);
    if (aligned && (a.cols & 3) == 0) return 0;
    return a.cols >= 4 ? 1 : 2;
}

// Workgroup w of nw zeroes its share of the padding rows [cbr, code_rows) of every batch of
// the code buffer (16-byte stores when the rows allow them), so no separate launch is needed.
template <int NT>
__device__ __forceinline__ void zero_pad_share(const scmp_quant_args &a, int64_t cbr, int64_t w,
                                               int64_t nw) {
    const int64_t pad_rows = a.code_rows - cbr;
    if (pad_rows <= 0) return;
    const int64_t nb = a.rows / cbr;
    const bool wide = (a.code_ld & 15) == 0 && ((uintptr_t)a.code & 15) == 0;
    const int64_t ub = wide ? 16 : 1;                      // bytes per unit
    const int64_t per = pad_rows * a.code_ld / ub;         // units per batch
    const int64_t total = per * nb;
    const int64_t u0 = total * w / nw, u1 = total * (w + 1) / nw;
    int64_t b = (u0 + threadIdx.x) / per;
    int64_t off = (u0 + threadIdx.x) - b * per;
    for (int64_t u = u0 + threadIdx.x; u < u1; u += NT) {
        uint8_t *dst = a.code + (b * a.code_rows + cbr) * a.code_ld + off * ub;
        if (wide) *(uint4 *)dst = make_uint4(0u, 0u, 0u, 0u);
        else *dst = 0;
        off += NT;
        while (off >= per) {
            off -= per;
            ++b;
        }
    }
}

// PT: register-held chunks per thread (npt <= PT); npt > PT re-reads the chunks instead.
template <int OP, int SM, int PT, int NT>
__global__ void __launch_bounds__(NT, NT == kMidGroupThreads ? 4 : 1)
quant_group_kernel(scmp_quant_args a, int G, int cpr, int npt) {
    __shared__ uint32_t red0[NT / 64], red1[NT / 64];
    __shared__ float rsums[kGroupMaxRows];
    __shared__ int64_t s_rowoff[kGroupMaxRows];
    __shared__ uint8_t s_jtab[256];
    constexpr bool SMOOTH = SM != SCMP_SMOOTH_NONE;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * G;
    const int nr = a.rows - r0 < G ? (int)(a.rows - r0) : G;
    const int nch = nr * cpr;                        // 4-column chunks of the group
    constexpr bool asym = OP == QOP_DIVZP;
    const bool want_sum = a.rowsum != nullptr;
    const bool thermo = a.code && a.code_kind == SCMP_CODE_THERMO;
    const bool lds_jtab = thermo && a.col_class == nullptr;
    // the thermometer table byte this thread places in LDS, loaded before any chunk (the
    // oldest load: waiting for it waits for no chunk); written after the chunks' loads
    const uint32_t jt = lds_jtab ? a.jtab[tid & 255] : 0u;
    // the caller's row index, staged in LDS as element offsets (one read per row, so that no
    // chunk load waits for its row's index); without one a row's start is computed
    const bool ridx = a.row_index != nullptr;
    if (ridx) {
        for (int i = tid; i < nr; i += NT) s_rowoff[i] = a.row_index[r0 + i] * a.ld;
        __syncthreads();
    }
    auto rowp = [&](int rr) __attribute__((always_inline)) {
        return a.x + (ridx ? s_rowoff[rr] : (r0 + rr) * a.ld);
    };
    // chunk loads (load_raw4): one 16-byte load, or four clamped 4-byte ones; a uniform
    // branch around a load whose value is used only after every load is issued
    const bool m0 = chunk_mode(a) == 0;
    auto load4 = [&](const float *row, int c, float (&t)[4]) __attribute__((always_inline)) {
        if (m0) load_raw4<0>(row, c, a.cols, t);
        else load_raw4<1>(row, c, a.cols, t);
    };

    // position (row, first column) of this thread's k-th chunk, chunk index tid + 256 k;
    // a step of 256 chunks is dr rows and dc chunks
    const int rr_first = tid / cpr;
    const int cc_first = tid - rr_first * cpr;
    const int dr = NT / cpr, dc = NT - dr * cpr;
    auto step_rows = [&](int &cc) __attribute__((always_inline)) {
        cc += dc;
        const bool wrap = cc >= cpr;
        if (wrap) cc -= cpr;
        return dr + (wrap ? 1 : 0);
    };
    auto advance = [&](int &rr, int &cc) __attribute__((always_inline)) {
        rr += step_rows(cc);
    };

    // pass 1: statistic of the group
    const bool reg = npt <= PT;
    float vals[PT][4];
    float mx = -INFINITY, mn = INFINITY, am = 0.0f;
    // Columns past the row end load as 0: harmless for max|x|, so only the asymmetric
    // statistic of a row whose last chunk is partial checks the column bound.
    const bool full = (a.cols & 3) == 0;
    auto fold = [&](const float (&v)[4], int c) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (asym && !full && c + k >= a.cols) break;
            if (asym) {
                mx = fmaxf(mx, v[k]);
                mn = fminf(mn, v[k]);
            } else {
                am = fmaxf(am, fabsf(v[k]));
            }
        }
    };
    float sv[SMOOTH ? PT : 1][4];
    // LDS tables written while the chunks' loads are in flight (read after the reduction's
    // barrier)
    auto write_tables = [&]() __attribute__((always_inline)) {
        if (want_sum)
            for (int i = tid; i < nr; i += NT) rsums[i] = 0.0f;
        if (lds_jtab && tid < 256) s_jtab[tid] = (uint8_t)jt;
    };
    if (reg) {
        // every load first (a lane past the group's chunks loads chunk 0), then the values
        int rr = rr_first, cc = cc_first;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const bool ok = k < npt && tid + k * NT < nch;
            const int lc = ok ? 4 * cc : 0;
            load4(rowp(ok ? rr : 0), lc, vals[k]);
            if (SMOOTH) load4(a.smooth, lc, sv[SMOOTH ? k : 0]);
            advance(rr, cc);
        }
        rr = rr_first;
        cc = cc_first;
        write_tables();
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            if (k < npt && tid + k * NT < nch) {
                finish4<1, SM>(4 * cc, a.cols, vals[k], sv[SMOOTH ? k : 0]);
                fold(vals[k], 4 * cc);
            }
            advance(rr, cc);
        }
    } else {
        write_tables();
        // four chunks per step, loads first
        int rr = rr_first, cc = cc_first;
        for (int ch = tid; ch < nch; ch += 4 * NT) {
            float v[4][4], s4[SMOOTH ? 4 : 1][4];
            int cu[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool ok = ch + u * NT < nch;
                cu[u] = 4 * cc;
                load4(rowp(ok ? rr : 0), ok ? 4 * cc : 0, v[u]);
                if (SMOOTH) load4(a.smooth, ok ? 4 * cc : 0, s4[SMOOTH ? u : 0]);
                advance(rr, cc);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (ch + u * NT < nch) {
                    finish4<1, SM>(cu[u], a.cols, v[u], s4[SMOOTH ? u : 0]);
                    fold(v[u], cu[u]);
                }
            }
        }
    }
    uint32_t k0, k1 = 0;
    if (asym) {
        mx = wave_max(mx);
        mn = wave_min(mn);
        k0 = key_of(mx);
        k1 = key_of(-mn);
    } else {
        k0 = __float_as_uint(wave_max(am));
    }
    if (lane == 0) {
        red0[wave] = k0;
        red1[wave] = k1;
    }
    __syncthreads();
    uint32_t s0 = red0[0], s1 = red1[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
        s0 = s0 > red0[w] ? s0 : red0[w];
        s1 = s1 > red1[w] ? s1 : red1[w];
    }
    const QParams p = derive_params(a, s0, asym ? s1 : 0u);

    // pass 2: codes and outputs
    const float qf = (float)a.q_max;
    const float qlo = asym ? 0.0f : (a.variant == SCMP_Q_HEAD_SYM ? -(qf + 1.0f) : -qf);
    const float rq = __fdiv_rn((float)a.rng_levels, qf);
    const float rf = (float)a.rng_levels;
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    const bool api_out = a.beta16 || a.beta32 || a.sign || a.xint;
    // Row sums: with rows of a multiple of 64 chunks (and NT a multiple of 64) the chunks of
    // one wave lie in one row and the wave is active as a whole, so it adds its sum with one
    // LDS atomic instead of 64 on the same address. Integer-valued: exact in any order.
    const bool wave_rows = cpr % 64 == 0;
    auto add_rowsum = [&](int rr, float qs) __attribute__((always_inline)) {
        if (wave_rows) {
            const float w = wave_sum(qs);
            if (lane == 0) atomicAdd(&rsums[rr], w);
        } else {
            atomicAdd(&rsums[rr], qs);
        }
    };
    // General element path: any chunk, any requested outputs.
    auto emit = [&](const float (&v)[4], int rr, int c) __attribute__((always_inline)) {
        const int64_t r = r0 + rr;
        uint32_t word = 0;
        float qs = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (c + k >= a.cols) break;
            const float t = OP == QOP_MUL ? rne(__fmul_rn(v[k], p.inv))
                                          : rne_quotient<OP>(v[k], p.s, p.inv, p.zp);
            const float q = fmin_first(fmax_first(t, qlo), qf);
            word |= (uint32_t)element_outputs(a, q, r, c + k, asym, rq, rf, qf) << (8 * k);
            qs += q;                                 // exact: integers below 2^24
        }
        if (a.code) {
            const int64_t b = r / cbr, i = r - b * cbr;
            *(uint32_t *)(a.code + (b * a.code_rows + i) * a.code_ld + c) = word;
        }
        if (want_sum) add_rowsum(rr, qs);
    };
    // Hot path: GEMM codes only (jtab in LDS, or per-column classes' rows of jtab read from
    // global memory). The four quotients take the
    // multiply-by-reciprocal route together; one branch per chunk redoes all four with
    // the exact division when any of them is within reach of a half-integer (see
    // rne_quotient for the bound).
    auto emit_fast = [&](const float (&v)[4], int rr, uint8_t *crow, int c)
        __attribute__((always_inline)) {
        float t[4];
        if (OP == QOP_MUL) {
#pragma unroll
            for (int k = 0; k < 4; ++k) t[k] = rne(__fmul_rn(v[k], p.inv));
        } else {
            bool ok = true;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float y = __fmul_rn(v[k], p.inv);
                const float u = OP == QOP_DIVZP ? __fadd_rn(y, p.zp) : y;
                t[k] = rne(u);
                ok = ok && __builtin_fabsf(y) < 1024.0f &&
                     __builtin_fabsf(__fsub_rn(u, t[k])) < 0.5f - 4.8828125e-4f;
            }
            if (!ok) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float e = __fdiv_rn(v[k], p.s);
                    t[k] = rne(OP == QOP_DIVZP ? __fadd_rn(e, p.zp) : e);
                }
            }
        }
        // columns past the row end (the last chunk of a row whose length is not a multiple
        // of 4) get code 0 and add nothing to the row sum
        const int nv = a.cols - c;
        uint32_t word = 0;
        float qs = 0.0f;
        // per-column table classes: the chunk's four classes (one 16-byte load for a full
        // chunk), each code from its class's row of jtab
        int cls[4] = {0, 0, 0, 0};
        if (thermo && !lds_jtab) {
            if (nv >= 4) {
                const int4 c4 = *(const int4 *)(a.col_class + c);
                cls[0] = c4.x; cls[1] = c4.y; cls[2] = c4.z; cls[3] = c4.w;
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) cls[k] = k < nv ? a.col_class[c + k] : 0;
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float q = k < nv ? fmin_first(fmax_first(t[k], qlo), qf) : 0.0f;
            const int qi = (int)q;
            uint32_t code;
            if (thermo) {
                const int mi = qi < 0 ? -qi : qi;
                code = lds_jtab ? s_jtab[mi] : a.jtab[(int64_t)cls[k] * 256 + mi];
                if (!asym && qi < 0) code |= 0x80u;
            } else {
                code = (uint32_t)(qi & 0xff);
            }
            word |= (k < nv ? code : 0u) << (8 * k);
            qs += q;
        }
        *(uint32_t *)(crow + c) = word;
        if (want_sum) add_rowsum(rr, qs);
    };
    // per-column classes are read with 16-byte loads: col_class 16-byte aligned
    const bool fast = !api_out && a.code &&
                      (lds_jtab || !thermo || ((uintptr_t)a.col_class & 15) == 0);
    if (fast) {
        // code row of input row r0 + rr: batch bb, row bi of the batch; tracked as rr grows
        // (a step that leaves a batch skips that batch's padding rows)
        const int64_t rf0 = r0 + rr_first;
        int64_t bb = rf0 / cbr, bi = rf0 - bb * cbr;
        uint8_t *crow = a.code + (bb * a.code_rows + bi) * a.code_ld;
        int rr = rr_first, cc = cc_first;
        auto advance_code = [&]() __attribute__((always_inline)) {
            const int n = step_rows(cc);
            rr += n;
            bi += n;
            crow += (int64_t)n * a.code_ld;
            while (bi >= cbr) {
                bi -= cbr;
                crow += (a.code_rows - cbr) * a.code_ld;
            }
        };
        if (reg) {
#pragma unroll
            for (int k = 0; k < PT; ++k) {
                if (k < npt && tid + k * NT < nch)
                    emit_fast(vals[k], rr, crow, 4 * cc);
                advance_code();
            }
        } else {
            for (int ch = tid; ch < nch; ch += 4 * NT) {
                float v[4][4], s4[SMOOTH ? 4 : 1][4];
                int ru[4], cu[4];
                uint8_t *cru[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool ok = ch + u * NT < nch;
                    ru[u] = rr;
                    cu[u] = 4 * cc;
                    cru[u] = crow;
                    load4(rowp(ok ? rr : 0), ok ? 4 * cc : 0, v[u]);
                    if (SMOOTH)
                        load4(a.smooth, ok ? 4 * cc : 0, s4[SMOOTH ? u : 0]);
                    advance_code();
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (ch + u * NT < nch) {
                        finish4<1, SM>(cu[u], a.cols, v[u], s4[SMOOTH ? u : 0]);
                        emit_fast(v[u], ru[u], cru[u], cu[u]);
                    }
                }
            }
        }
    } else if (reg) {
        int rr = rr_first, cc = cc_first;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            if (k < npt && tid + k * NT < nch) emit(vals[k], rr, 4 * cc);
            advance(rr, cc);
        }
    } else {
        int rr = rr_first, cc = cc_first;
        for (int ch = tid; ch < nch; ch += 4 * NT) {
            float v[4][4], s4[SMOOTH ? 4 : 1][4];
            int ru[4], cu[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool ok = ch + u * NT < nch;
                ru[u] = rr;
                cu[u] = 4 * cc;
                load4(rowp(ok ? rr : 0), ok ? 4 * cc : 0, v[u]);
                if (SMOOTH) load4(a.smooth, ok ? 4 * cc : 0, s4[SMOOTH ? u : 0]);
                advance(rr, cc);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (ch + u * NT < nch) {
                    finish4<1, SM>(cu[u], a.cols, v[u], s4[SMOOTH ? u : 0]);
                    emit(v[u], ru[u], cu[u]);
                }
            }
        }
    }
    // zero code columns past the last 4-column chunk, per row of the group
    if (a.code) {
        const int c0 = 4 * cpr;
        const int tail = (int)(a.code_ld - c0);
        for (int e = tid; e < nr * tail; e += NT) {
            const int rr = e / tail, c = c0 + (e - rr * tail);
            const int64_t r = r0 + rr, b = r / cbr, i = r - b * cbr;
            a.code[(b * a.code_rows + i) * a.code_ld + c] = 0;
        }
    }
    if (a.code) zero_pad_share<NT>(a, cbr, blockIdx.x, gridDim.x);
    __syncthreads();
    for (int rr = tid; rr < nr; rr += NT) {
        const int64_t r = r0 + rr;
        if (a.scale) a.scale[r] = p.s;
        if (a.inv) a.inv[r] = p.inv;
        if (a.zp) a.zp[r] = p.zp;
        if (want_sum) a.rowsum[r] = rsums[rr];
    }
}

// ---------------------------------------------------------------------------------
// Lean one-pass group quantizer for the common case of the SC matmul: GEMM codes only (no
// boundary / sign / integer outputs), thermometer codes from one table (jtab in LDS) or the
// quantized integers as bytes, every chunk of the group held in registers. Same statistic,
// parameters and per-element operations as quant_group_kernel, with the element path cut
// to a few instructions: the code byte of q comes from one 512-entry LDS table indexed by
// q (sign bit included), the clamp runs on the integer (equal for integer-valued rounded
// quotients, NaN included: it converts to 0 either way), and the four code bytes of a chunk
// are packed by shifts. CODE: SCMP_CODE_THERMO or SCMP_CODE_Q; SUM: row sums (zero-point
// variant; the clamp then also runs in fp32, as the row sum adds the fp32 value). The load
// mode and the smoothing are uniform branches around loads whose values are used only
// after every load is issued.
// ---------------------------------------------------------------------------------
// DENSE: x rows, code rows and the group all contiguous (ld = code_ld = cols, a multiple of
// 4, 16-byte aligned; no row index; no group across a batch): chunk k of a thread is chunk
// tid + k * NT of the group in both buffers, so its addresses are fixed offsets.
// blk: the group (row block) this workgroup quantizes, nblk: the groups of the call.
template <int OP, int PT, int NT, int CODE, bool SUM, bool SMOOTH, bool DENSE>
__device__ __forceinline__ void quant_codes_body(const scmp_quant_args &a, int G, int cpr,
                                                 int npt, int blk, int nblk) {
    __shared__ uint32_t red0[NT / 64], red1[NT / 64];
    __shared__ float rsums[SUM ? kGroupMaxRows : 1];
    __shared__ int64_t s_rowoff[kGroupMaxRows];
    __shared__ uint8_t s_code[CODE == SCMP_CODE_THERMO ? 512 : 1];
    constexpr bool asym = OP == QOP_DIVZP;
    const int sm = SMOOTH ? a.smooth_mode : SCMP_SMOOTH_NONE;
    const bool m0 = chunk_mode(a) == 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t r0 = (int64_t)blk * G;
    const int nr = a.rows - r0 < G ? (int)(a.rows - r0) : G;
    const int nch = nr * cpr;
    const int qmax = a.q_max;
    const int qlo = asym ? 0 : (a.variant == SCMP_Q_HEAD_SYM ? -(qmax + 1) : -qmax);
    // the caller's row index, staged in LDS (one read per row); without one, a row's start
    // is computed and the loads go out before any table is built
    const bool ridx = a.row_index != nullptr;
    if (ridx) {
        for (int i = tid; i < nr; i += NT) s_rowoff[i] = a.row_index[r0 + i] * a.ld;
        __syncthreads();
    }
    auto rowp = [&](int rr) __attribute__((always_inline)) {
        return a.x + (ridx ? s_rowoff[rr] : (r0 + rr) * a.ld);
    };

    const int rr_first = tid / cpr;
    const int cc_first = tid - rr_first * cpr;
    const int dr = NT / cpr, dc = NT - dr * cpr;
    auto advance = [&](int &rr, int &cc) __attribute__((always_inline)) {
        cc += dc;
        const bool wrap = cc >= cpr;
        if (wrap) cc -= cpr;
        rr += dr + (wrap ? 1 : 0);
    };
    // a chunk's element offset within the group's rows of x (ld apart) and of the codes
    // (code_ld apart), tracked in 32 bits from the group's first row (groups hold fewer
    // than 2^22 elements)
    const uint32_t ld32 = (uint32_t)a.ld, cld32 = (uint32_t)a.code_ld;
    const uint32_t xstep = (uint32_t)dr * ld32 + 4u * (uint32_t)dc, xwrap = ld32 - 4u * (uint32_t)cpr;
    const uint32_t cstep = (uint32_t)dr * cld32 + 4u * (uint32_t)dc, cwrap = cld32 - 4u * (uint32_t)cpr;
    auto advance_off = [&](int &rr, int &cc, uint32_t &xo, uint32_t &co)
        __attribute__((always_inline)) {
        cc += dc;
        const bool wrap = cc >= cpr;
        if (wrap) cc -= cpr;
        rr += dr + (wrap ? 1 : 0);
        xo += xstep + (wrap ? xwrap : 0u);
        co += cstep + (wrap ? cwrap : 0u);
    };
    const float *xg = a.x + r0 * a.ld;                  // the group's first row (no row index)

    // the thermometer table entries this thread will place in the code table, loaded first
    // (the oldest load, so waiting for it waits for no chunk) with clamped indices
    constexpr int NTAB = CODE == SCMP_CODE_THERMO ? (512 + NT - 1) / NT : 1;
    uint32_t jt[NTAB];
    if (CODE == SCMP_CODE_THERMO) {
#pragma unroll
        for (int j = 0; j < NTAB; ++j) {
            const int q = (tid + j * NT) - 256;
            const int m = q < 0 ? -q : q;
            jt[j] = a.jtab[m < 255 ? m : 255];
        }
    }
    // pass 1: every load, then the statistic
    float vals[PT][4];
    float sv[SMOOTH ? PT : 1][4];
    {
        int rr = rr_first, cc = cc_first;
        uint32_t xo = (uint32_t)rr_first * ld32 + 4u * (uint32_t)cc_first, co = 0;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            const bool ok = k < npt && tid + k * NT < nch;
            const int lc = ok ? 4 * cc : 0;
            if (DENSE) {
                const float4 x4 = ((const float4 *)(a.x + r0 * a.cols))[ok ? tid + k * NT : 0];
                vals[k][0] = x4.x; vals[k][1] = x4.y; vals[k][2] = x4.z; vals[k][3] = x4.w;
                if (SMOOTH) load_raw4<0>(a.smooth, lc, a.cols, sv[SMOOTH ? k : 0]);
            } else {
                const float *row = ridx ? rowp(ok ? rr : 0) : xg + (ok ? xo - 4u * (uint32_t)cc : 0u);
                if (m0) load_raw4<0>(row, lc, a.cols, vals[k]);
                else load_raw4<1>(row, lc, a.cols, vals[k]);
                if (SMOOTH) {
                    if (m0) load_raw4<0>(a.smooth, lc, a.cols, sv[SMOOTH ? k : 0]);
                    else load_raw4<1>(a.smooth, lc, a.cols, sv[SMOOTH ? k : 0]);
                }
            }
            if (DENSE) {
                if (SMOOTH || SUM) advance(rr, cc);
            } else {
                advance_off(rr, cc, xo, co);
            }
        }
    }
    // while the loads are in flight: row sums and the code table (read after the
    // reduction's barrier)
    if (SUM)
        for (int i = tid; i < nr; i += NT) rsums[i] = 0.0f;
    if (CODE == SCMP_CODE_THERMO) {
        // code byte of q = i - 256 for the q the clamp lets through
#pragma unroll
        for (int j = 0; j < NTAB; ++j) {
            const int i = tid + j * NT;
            const int q = i - 256;
            uint32_t c = (q >= qlo && q <= qmax) ? jt[j] : 0u;
            if (!asym && q < 0) c |= 0x80u;
            if (i < 512) s_code[i] = (uint8_t)c;
        }
    }
    float mx = -INFINITY, mn = INFINITY, am = 0.0f;
    const bool full = (a.cols & 3) == 0;
    {
        int rr = rr_first, cc = cc_first;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            if (k < npt && tid + k * NT < nch) {
                const int c = 4 * cc;
                float (&svk)[4] = sv[SMOOTH ? k : 0];
                if (SMOOTH && sm == SCMP_SMOOTH_DIV) finish4<1, SCMP_SMOOTH_DIV>(c, a.cols, vals[k], svk);
                else if (SMOOTH && sm == SCMP_SMOOTH_MUL) finish4<1, SCMP_SMOOTH_MUL>(c, a.cols, vals[k], svk);
                else if (!DENSE) finish4<1, SCMP_SMOOTH_NONE>(c, a.cols, vals[k], svk);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (asym && !DENSE && !full && c + e >= a.cols) break;
                    if (asym) {
                        mx = fmaxf(mx, vals[k][e]);
                        mn = fminf(mn, vals[k][e]);
                    } else {
                        am = fmaxf(am, fabsf(vals[k][e]));
                    }
                }
            }
            if (!DENSE || SMOOTH || SUM) advance(rr, cc);
        }
    }
    uint32_t k0, k1 = 0;
    if (asym) {
        mx = wave_max(mx);
        mn = wave_min(mn);
        k0 = key_of(mx);
        k1 = key_of(-mn);
    } else {
        k0 = __float_as_uint(wave_max(am));
    }
    if (lane == 0) {
        red0[wave] = k0;
        red1[wave] = k1;
    }
    __syncthreads();
    uint32_t s0 = red0[0], s1 = red1[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) {
        s0 = s0 > red0[w] ? s0 : red0[w];
        s1 = s1 > red1[w] ? s1 : red1[w];
    }
    const QParams p = derive_params(a, s0, asym ? s1 : 0u);

    // pass 2: the code word of every chunk
    const float qf = (float)qmax, qlof = (float)qlo;
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    const bool wave_rows = cpr % 64 == 0;
    {
        // DENSE: the group's first code row (r0's batch and row within it)
        const int64_t gb = r0 / cbr;
        uint32_t *cg = (uint32_t *)(a.code + (gb * a.code_rows + (r0 - gb * cbr)) * a.code_ld);
        // the pass restarts from an opaque copy of the first position, so the chunk
        // offsets are recomputed here instead of kept in registers from the first pass
        int rr = rr_first, cc = cc_first;
        asm volatile("" : "+v"(rr), "+v"(cc));
        uint32_t xo = 0, co = (uint32_t)rr * cld32 + 4u * (uint32_t)cc;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
            if (k < npt && tid + k * NT < nch) {
                const int c = 4 * cc;
                const float (&v)[4] = vals[k];
                float t[4];
                if (OP == QOP_MUL) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] = rne(__fmul_rn(v[e], p.inv));
                } else {
                    bool ok = true;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float y = __fmul_rn(v[e], p.inv);
                        const float u = OP == QOP_DIVZP ? __fadd_rn(y, p.zp) : y;
                        t[e] = rne(u);
                        ok = ok && __builtin_fabsf(y) < 1024.0f &&
                             __builtin_fabsf(__fsub_rn(u, t[e])) < 0.5f - 4.8828125e-4f;
                    }
                    if (!ok) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float d = __fdiv_rn(v[e], p.s);
                            t[e] = rne(OP == QOP_DIVZP ? __fadd_rn(d, p.zp) : d);
                        }
                    }
                }
                const int nv = DENSE ? 4 : a.cols - c;
                uint32_t word = 0;
                float qs = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int qi = (int)t[e];
                    qi = qi < qlo ? qlo : (qi > qmax ? qmax : qi);
                    uint32_t code;
                    if (CODE == SCMP_CODE_THERMO) code = s_code[qi + 256];
                    else code = (uint32_t)(qi & 0xff);
                    word |= (e < nv ? code : 0u) << (8 * e);
                    if (SUM) qs += e < nv ? fmin_first(fmax_first(t[e], qlof), qf) : 0.0f;
                }
                if (DENSE) cg[tid + k * NT] = word;
                else *(uint32_t *)((uint8_t *)cg + co) = word;
                if (SUM) {
                    if (wave_rows) {
                        const float w = wave_sum(qs);
                        if (lane == 0) atomicAdd(&rsums[rr], w);
                    } else {
                        atomicAdd(&rsums[rr], qs);
                    }
                }
            }
            // next chunk's row: the code row follows, skipping a batch's padding rows
            if (DENSE) {
                if (SUM) advance(rr, cc);
            } else {
                advance_off(rr, cc, xo, co);
            }
        }
    }
    // code columns past the last 4-column chunk, and the batches' padding rows
    {
        const int c0 = 4 * cpr;
        const int tail = (int)(a.code_ld - c0);
        for (int e = tid; e < nr * tail; e += NT) {
            const int rr = e / tail, c = c0 + (e - rr * tail);
            const int64_t r = r0 + rr, b = r / cbr, i = r - b * cbr;
            a.code[(b * a.code_rows + i) * a.code_ld + c] = 0;
        }
    }
    zero_pad_share<NT>(a, cbr, blk, nblk);
    if (SUM) __syncthreads();
    for (int rr = tid; rr < nr; rr += NT) {
        const int64_t r = r0 + rr;
        if (a.scale) a.scale[r] = p.s;
        if (a.inv) a.inv[r] = p.inv;
        if (a.zp) a.zp[r] = p.zp;
        if (SUM) a.rowsum[r] = rsums[rr];
    }
}

template <int OP, int PT, int NT, int CODE, bool SUM, bool SMOOTH, bool DENSE>
__global__ void __launch_bounds__(NT, NT == kMidGroupThreads ? 4 : 1)
quant_codes_kernel(scmp_quant_args a, int G, int cpr, int npt) {
    quant_codes_body<OP, PT, NT, CODE, SUM, SMOOTH, DENSE>(a, G, cpr, npt, blockIdx.x, gridDim.x);
}

// Two calls of the same shape class in one launch (an attention call's q and k): the first
// n1 workgroups quantize a's groups (thermometer codes), the rest b's (byte codes), so the
// two calls' load latencies overlap instead of running one launch after the other.
template <int OP, int PT, int NT, bool DENSE>
__global__ void __launch_bounds__(NT, 1)
quant_codes_pair_kernel(scmp_quant_args a, scmp_quant_args b, int n1, int G1, int cpr1,
                        int npt1, int G2, int cpr2, int npt2) {
    const int blk = (int)blockIdx.x;
    if (blk < n1)
        quant_codes_body<OP, PT, NT, SCMP_CODE_THERMO, false, false, DENSE>(a, G1, cpr1, npt1, blk, n1);
    else
        quant_codes_body<OP, PT, NT, SCMP_CODE_Q, false, false, DENSE>(
            b, G2, cpr2, npt2, blk - n1, (int)gridDim.x - n1);
}

template <int OP, int PT, int NT>
static void launch_codes(const scmp_quant_args &a, dim3 grid, int G, int cpr, int npt,
                         hipStream_t stream) {
    constexpr bool SUM = OP == QOP_DIVZP;
    const bool th = a.code_kind == SCMP_CODE_THERMO;
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    const bool dense = chunk_mode(a) == 0 && a.ld == a.cols && a.code_ld == a.cols &&
                       !a.row_index && cbr % G == 0;
#define SCMP_LAUNCH_CODES(SMOOTH, DENSE)                                                      \
    do {                                                                                     \
        if (th)                                                                              \
            quant_codes_kernel<OP, PT, NT, SCMP_CODE_THERMO, SUM, SMOOTH, DENSE>             \
                <<<grid, NT, 0, stream>>>(a, G, cpr, npt);                                   \
        else                                                                                 \
            quant_codes_kernel<OP, PT, NT, SCMP_CODE_Q, SUM, SMOOTH, DENSE>                  \
                <<<grid, NT, 0, stream>>>(a, G, cpr, npt);                                   \
    } while (0)
    if (a.smooth_mode != SCMP_SMOOTH_NONE) {
        if (dense) SCMP_LAUNCH_CODES(true, true);
        else SCMP_LAUNCH_CODES(true, false);
    } else {
        if (dense) SCMP_LAUNCH_CODES(false, true);
        else SCMP_LAUNCH_CODES(false, false);
    }
#undef SCMP_LAUNCH_CODES
}

// The lean kernel's launch for a call it covers (codes only, one thermometer table or byte
// codes, row sums exactly for the zero-point variant, every chunk in registers); false:
// not covered.
template <int OP>
static bool try_codes(const scmp_quant_args &a, dim3 grid, int G, int cpr, int npt, int wide,
                      hipStream_t stream) {
    if (!a.code || a.beta16 || a.beta32 || a.sign || a.xint || a.cols < 4) return false;
    if (a.code_kind == SCMP_CODE_THERMO && a.col_class != nullptr) return false;
    if ((a.rowsum != nullptr) != (OP == QOP_DIVZP)) return false;
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    if (cbr % G != 0 && cbr < a.rows) return false;      // a group across a batch boundary
    if (wide == 1) {
        launch_codes<OP, 4, kBigGroupThreads>(a, grid, G, cpr,
                                              (int)cdiv((int64_t)G * cpr, kBigGroupThreads), stream);
    } else if (wide == 2) {
        launch_codes<OP, 8, kMidGroupThreads>(a, grid, G, cpr,
                                              (int)cdiv((int64_t)G * cpr, kMidGroupThreads), stream);
    } else if (npt <= 4) {
        launch_codes<OP, 4, kGroupThreads>(a, grid, G, cpr, npt, stream);
    } else if (npt <= kMaxChunks) {
        launch_codes<OP, kMaxChunks, kGroupThreads>(a, grid, G, cpr, npt, stream);
    } else if (OP == QOP_MUL && a.smooth_mode == SCMP_SMOOTH_NONE && chunk_mode(a) != 2 &&
               cdiv((int64_t)G * cpr, kMidGroupThreads) <= kMidChunks) {
        // groups of 4097 to 10240 chunks without smoothing (an attention head's P): 512
        // threads, two workgroups per compute unit, so two groups overlap their loads and
        // their code writes (one 1024-thread workgroup per compute unit would run the groups
        // in lockstep rounds); the general chunk path, which takes any row layout
        const int npt2 = (int)cdiv((int64_t)G * cpr, kMidGroupThreads);
        if (a.code_kind == SCMP_CODE_THERMO)
            quant_codes_kernel<QOP_MUL, kMidChunks, kMidGroupThreads, SCMP_CODE_THERMO, false,
                               false, false><<<grid, kMidGroupThreads, 0, stream>>>(a, G, cpr, npt2);
        else
            quant_codes_kernel<QOP_MUL, kMidChunks, kMidGroupThreads, SCMP_CODE_Q, false, false,
                               false><<<grid, kMidGroupThreads, 0, stream>>>(a, G, cpr, npt2);
    } else if (OP == QOP_MUL && cdiv((int64_t)G * cpr, kBigGroupThreads) <= kBigChunks) {
        launch_codes<QOP_MUL, kBigChunks, kBigGroupThreads>(
            a, grid, G, cpr, (int)cdiv((int64_t)G * cpr, kBigGroupThreads), stream);
    } else {
        return false;
    }
    return true;
}

// Zero the padding rows [code_batch_rows, code_rows) of every batch of a code buffer.
__global__ void zero_code_rows_kernel(uint8_t *code, int64_t ld, int64_t code_rows,
                                      int64_t cbr, int64_t nbatch) {
    const int64_t per = (code_rows - cbr) * ld;
    const int64_t total = per * nbatch;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = e / per, off = e - b * per;
        code[(b * code_rows + cbr) * ld + off] = 0;
    }
}

__global__ void tensor_out_kernel(const QParams *prm, double *scale64, double *zp64) {
    if (scale64) scale64[0] = prm[0].s64;
    if (zp64) zp64[0] = prm[0].zp64;
}

static inline void unit_counts(int64_t rows, int64_t cols, int64_t group, int64_t seg,
                               int64_t *g, int64_t *segw, int64_t *nseg) {
    int64_t G = group <= 0 || group > rows ? rows : group;
    *g = G;
    *segw = seg > 0 && seg < cols ? seg : (cols > 0 ? cols : 1);
    *nseg = cdiv(cols > 0 ? cols : 1, *segw);
}

// ---------------------------------------------------------------------------------
// One-pass quantizer for one-row groups split into column segments (chunk_d): one
// 256-thread workgroup per row keeps the row in registers; every 4-column chunk lies in
// one segment (segment width a multiple of 4), folds its statistic into the segment's
// LDS slot with the same order-independent atomic max as reduce_kernel, and the segment
// parameters are derived once per segment in LDS.
// ---------------------------------------------------------------------------------

constexpr int kMaxSegs = 256;

template <int OP, int SM, int PT>
__global__ void __launch_bounds__(kGroupThreads)
quant_seg_kernel(scmp_quant_args a, int cpr, int segw, int nseg) {
    __shared__ uint32_t s_st0[kMaxSegs], s_st1[kMaxSegs];
    __shared__ QParams s_prm[kMaxSegs];
    __shared__ uint8_t s_jtab[256];
    __shared__ float s_rsum;
    const int tid = threadIdx.x;
    const int64_t r = blockIdx.x;
    constexpr bool asym = OP == QOP_DIVZP;
    const bool thermo = a.code && a.code_kind == SCMP_CODE_THERMO;
    const bool lds_jtab = thermo && a.col_class == nullptr;
    // the thermometer table byte of this thread, loaded before any chunk (see below)
    const uint32_t jt = lds_jtab ? a.jtab[tid] : 0u;

    constexpr bool SMOOTH = SM != SCMP_SMOOTH_NONE;
    const float *xr = x_row(a, r);
    const bool m0 = chunk_mode(a) == 0;
    float vals[PT][4];
    float sv[SMOOTH ? PT : 1][4];
    // every load first (a lane past the row's chunks loads chunk 0), then the values
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const int cc = tid + k * kGroupThreads;
        const int lc = cc < cpr ? 4 * cc : 0;
        if (m0) load_raw4<0>(xr, lc, a.cols, vals[k]);
        else load_raw4<1>(xr, lc, a.cols, vals[k]);
        if (SMOOTH) {
            if (m0) load_raw4<0>(a.smooth, lc, a.cols, sv[SMOOTH ? k : 0]);
            else load_raw4<1>(a.smooth, lc, a.cols, sv[SMOOTH ? k : 0]);
        }
    }
    // LDS state, set up while the loads are in flight
    for (int t = tid; t < nseg; t += kGroupThreads) s_st0[t] = s_st1[t] = 0u;
    if (lds_jtab) s_jtab[tid] = (uint8_t)jt;
    if (tid == 0) s_rsum = 0.0f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const int cc = tid + k * kGroupThreads;
        if (cc < cpr) {
            const int c = 4 * cc;
            finish4<1, SM>(c, a.cols, vals[k], sv[SMOOTH ? k : 0]);
            float mx = -INFINITY, mn = INFINITY, am = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (c + e >= a.cols) break;
                if (asym) {
                    mx = fmaxf(mx, vals[k][e]);
                    mn = fminf(mn, vals[k][e]);
                } else {
                    am = fmaxf(am, fabsf(vals[k][e]));
                }
            }
            const int sg = (unsigned)c / (unsigned)segw;
            if (asym) {
                atomicMax(&s_st0[sg], key_of(mx));
                atomicMax(&s_st1[sg], key_of(-mn));
            } else {
                atomicMax(&s_st0[sg], __float_as_uint(am));
            }
        }
    }
    __syncthreads();
    for (int t = tid; t < nseg; t += kGroupThreads)
        s_prm[t] = derive_params(a, s_st0[t], asym ? s_st1[t] : 0u);
    __syncthreads();

    const float qf = (float)a.q_max;
    const float qlo = asym ? 0.0f : (a.variant == SCMP_Q_HEAD_SYM ? -(qf + 1.0f) : -qf);
    const float rq = __fdiv_rn((float)a.rng_levels, qf);
    const float rf = (float)a.rng_levels;
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    const int64_t bb = r / cbr, bi = r - bb * cbr;
    uint8_t *crow = a.code ? a.code + (bb * a.code_rows + bi) * a.code_ld : nullptr;
    const bool api_out = a.beta16 || a.beta32 || a.sign || a.xint;
    const bool fast = !api_out && a.code && !(thermo && !lds_jtab);
    float qs = 0.0f;
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const int cc = tid + k * kGroupThreads;
        if (cc < cpr) {
            const int c = 4 * cc;
            const QParams &p = s_prm[(unsigned)c / (unsigned)segw];
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (c + e >= a.cols) break;
                const float t = OP == QOP_MUL ? rne(__fmul_rn(vals[k][e], p.inv))
                                              : rne_quotient<OP>(vals[k][e], p.s, p.inv, p.zp);
                const float q = fmin_first(fmax_first(t, qlo), qf);
                uint32_t code;
                if (fast) {
                    const int qi = (int)q;
                    if (thermo) {
                        code = s_jtab[qi < 0 ? -qi : qi];
                        if (!asym && qi < 0) code |= 0x80u;
                    } else {
                        code = (uint32_t)(qi & 0xff);
                    }
                } else {
                    code = element_outputs(a, q, r, c + e, asym, rq, rf, qf);
                }
                word |= code << (8 * e);
                qs += q;                             // exact: integers below 2^24
            }
            if (crow) *(uint32_t *)(crow + c) = word;
        }
    }
    if (crow)
        for (int64_t c = 4 * (int64_t)cpr + tid; c < a.code_ld; c += kGroupThreads) crow[c] = 0;
    if (a.rowsum) atomicAdd(&s_rsum, qs);
    __syncthreads();
    for (int t = tid; t < nseg; t += kGroupThreads) {
        if (a.scale) a.scale[(int64_t)t * a.rows + r] = s_prm[t].s;
        if (a.inv) a.inv[(int64_t)t * a.rows + r] = s_prm[t].inv;
    }
    if (tid == 0) {
        if (a.zp) a.zp[r] = s_prm[0].zp;
        if (a.rowsum) a.rowsum[r] = s_rsum;
    }
}

template <int OP, int PT>
static void launch_seg_pt(const scmp_quant_args &a, int cpr, int segw, int nseg,
                          hipStream_t stream) {
    const dim3 grid((unsigned)a.rows);
    switch (a.smooth_mode) {
    case SCMP_SMOOTH_DIV:
        quant_seg_kernel<OP, SCMP_SMOOTH_DIV, PT><<<grid, kGroupThreads, 0, stream>>>(
            a, cpr, segw, nseg);
        break;
    case SCMP_SMOOTH_MUL:
        quant_seg_kernel<OP, SCMP_SMOOTH_MUL, PT><<<grid, kGroupThreads, 0, stream>>>(
            a, cpr, segw, nseg);
        break;
    default:
        quant_seg_kernel<OP, SCMP_SMOOTH_NONE, PT><<<grid, kGroupThreads, 0, stream>>>(
            a, cpr, segw, nseg);
        break;
    }
}

// One-row groups with column segments: the row (up to 16384 columns) in registers.
static int quantize_segments(const scmp_quant_args &a, int64_t segw, int64_t nseg,
                             hipStream_t stream) {
    const int cpr = (int)cdiv(a.cols, 4);
    const bool small = cpr <= 4 * kGroupThreads;
    switch (a.variant) {
    case SCMP_Q_GROUP_SYM:
        if (small) launch_seg_pt<QOP_DIV, 4>(a, cpr, (int)segw, (int)nseg, stream);
        else launch_seg_pt<QOP_DIV, kMaxChunks>(a, cpr, (int)segw, (int)nseg, stream);
        break;
    case SCMP_Q_GROUP_ASYM:
        if (small) launch_seg_pt<QOP_DIVZP, 4>(a, cpr, (int)segw, (int)nseg, stream);
        else launch_seg_pt<QOP_DIVZP, kMaxChunks>(a, cpr, (int)segw, (int)nseg, stream);
        break;
    default:
        if (small) launch_seg_pt<QOP_MUL, 4>(a, cpr, (int)segw, (int)nseg, stream);
        else launch_seg_pt<QOP_MUL, kMaxChunks>(a, cpr, (int)segw, (int)nseg, stream);
        break;
    }
    SCMP_LAUNCH_CHECK("scmp_quantize/segments");
    if (a.code) {
        const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
        if (a.code_rows > cbr) {
            const int64_t total = (a.code_rows - cbr) * a.code_ld * (a.rows / cbr);
            int64_t blocks = cdiv(total, 256);
            if (blocks > 4096) blocks = 4096;
            zero_code_rows_kernel<<<blocks, 256, 0, stream>>>(a.code, a.code_ld, a.code_rows,
                                                              cbr, a.rows / cbr);
            SCMP_LAUNCH_CHECK("scmp_quantize/pad");
        }
    }
    return SCMP_OK;
}

// One workgroup per row group, instantiated for the variant's element operation, the
// smoothing mode and the register-held chunk count (4: rows up to 4096 columns; 16).
template <int OP, int PT, int NT = kGroupThreads>
static void launch_group_pt(const scmp_quant_args &a, dim3 grid, int G, int cpr, int npt,
                            hipStream_t stream) {
    switch (a.smooth_mode) {
    case SCMP_SMOOTH_DIV:
        quant_group_kernel<OP, SCMP_SMOOTH_DIV, PT, NT><<<grid, NT, 0, stream>>>(a, G, cpr, npt);
        break;
    case SCMP_SMOOTH_MUL:
        quant_group_kernel<OP, SCMP_SMOOTH_MUL, PT, NT><<<grid, NT, 0, stream>>>(a, G, cpr, npt);
        break;
    default:
        quant_group_kernel<OP, SCMP_SMOOTH_NONE, PT, NT><<<grid, NT, 0, stream>>>(a, G, cpr, npt);
        break;
    }
}

// A group too large for 256 threads' registers takes 1024 threads (multiply-by-reciprocal
// variants: the per-head attention operands, one group per head), so it is read once.
// `wide`: few groups of 1025 to 4096 chunks (a row subset of a mixed-precision level)
// also take more threads, more loads in flight per group: 1024 (wide 1) when the groups fit
// the compute units once, else 512 (wide 2), two workgroups per compute unit, so that every
// group is in flight at once.
template <int OP>
static void launch_group(const scmp_quant_args &a, dim3 grid, int G, int cpr, int npt,
                         int wide, hipStream_t stream) {
    if (wide == 1) {
        launch_group_pt<OP, 4, kBigGroupThreads>(a, grid, G, cpr,
                                                 (int)cdiv((int64_t)G * cpr, kBigGroupThreads),
                                                 stream);
    } else if (wide == 2) {
        launch_group_pt<OP, 8, kMidGroupThreads>(a, grid, G, cpr,
                                                 (int)cdiv((int64_t)G * cpr, kMidGroupThreads),
                                                 stream);
    } else if (npt <= 4) {
        launch_group_pt<OP, 4>(a, grid, G, cpr, npt, stream);
    } else if (npt <= kMaxChunks || OP != QOP_MUL) {
        launch_group_pt<OP, kMaxChunks>(a, grid, G, cpr, npt, stream);
    } else {
        const int64_t per = cdiv((int64_t)G * cpr, kBigGroupThreads);
        const int npt4 = (int)(per <= kBigChunks ? per : kBigChunks + 1);
        launch_group_pt<QOP_MUL, kBigChunks, kBigGroupThreads>(a, grid, G, cpr, npt4, stream);
    }
}

// Compute units of the current device (cached per device).
static int quant_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

static int quantize_groups(const scmp_quant_args &a, int64_t G, hipStream_t stream) {
    const int64_t ngroups = cdiv(a.rows, G);
    const int64_t cpr = cdiv(a.cols, 4);
    // fewer than two 256-thread workgroups per compute unit, each group one to four chunks
    // per thread at 1024 threads (or two to eight at 512, when there are more groups than
    // compute units)
    const int64_t ncu = quant_cu_count();
    const int wide = ngroups < 2 * ncu && G * cpr > kBigGroupThreads &&
                             G * cpr <= 4 * (int64_t)kBigGroupThreads
                         ? (ngroups > ncu ? 2 : 1)
                         : 0;
    const int64_t per = cdiv(G * cpr, kGroupThreads);
    const dim3 grid((unsigned)ngroups);
    const int npt = (int)(per <= kMaxChunks ? per : kMaxChunks + 1);   // at 256 threads
    switch (a.variant) {
    case SCMP_Q_GROUP_SYM:
        if (!try_codes<QOP_DIV>(a, grid, (int)G, (int)cpr, npt, wide, stream))
            launch_group<QOP_DIV>(a, grid, (int)G, (int)cpr, npt, wide, stream);
        break;
    case SCMP_Q_GROUP_ASYM:
        if (!try_codes<QOP_DIVZP>(a, grid, (int)G, (int)cpr, npt, wide, stream))
            launch_group<QOP_DIVZP>(a, grid, (int)G, (int)cpr, npt, wide, stream);
        break;
    default:
        if (!try_codes<QOP_MUL>(a, grid, (int)G, (int)cpr, npt, wide, stream))
            launch_group<QOP_MUL>(a, grid, (int)G, (int)cpr, npt, wide, stream);
        break;
    }
    SCMP_LAUNCH_CHECK("scmp_quantize/group");   // the kernels zero the padding rows too
    return SCMP_OK;
}

// The argument checks of one quantizer call.
static int check_quant_args(const scmp_quant_args &a) {
    SCMP_REQUIRE(a.x && a.rows > 0 && a.cols > 0 && a.ld >= a.cols,
                 "scmp_quantize: bad input shape rows=%lld cols=%lld ld=%lld",
                 (long long)a.rows, (long long)a.cols, (long long)a.ld);
    SCMP_REQUIRE(a.variant >= SCMP_Q_GROUP_SYM && a.variant <= SCMP_Q_HOST_ASYM,
                 "scmp_quantize: unknown variant %d", a.variant);
    SCMP_REQUIRE(a.q_max >= 1 && a.q_max < (1 << 24), "scmp_quantize: q_max=%d out of range",
                 a.q_max);
    SCMP_REQUIRE(!a.code || a.q_max <= 255,
                 "scmp_quantize: GEMM codes need q_max <= 255 (got %d)", a.q_max);
    SCMP_REQUIRE(a.workspace != nullptr, "scmp_quantize: workspace required");
    SCMP_REQUIRE(a.smooth_mode == SCMP_SMOOTH_NONE || a.smooth != nullptr,
                 "scmp_quantize: smooth_mode set without smooth vector");
    if (a.code) {
        const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
        SCMP_REQUIRE(a.rows % cbr == 0, "scmp_quantize: rows %lld not a multiple of the "
                     "batch rows %lld", (long long)a.rows, (long long)cbr);
        // codes are written as 4-byte words per 4-column chunk
        SCMP_REQUIRE(a.code_ld >= 4 * cdiv(a.cols, 4) && a.code_rows >= cbr,
                     "scmp_quantize: code buffer rows/ld (%lld, %lld) smaller than the input "
                     "(ld must cover cols rounded up to 4)",
                     (long long)a.code_rows, (long long)a.code_ld);
        SCMP_REQUIRE(a.code_kind == SCMP_CODE_Q || (a.code_kind == SCMP_CODE_THERMO && a.jtab),
                     "scmp_quantize: THERMO codes need jtab");
    }
    if (a.beta16 || a.beta32 || a.sign || a.xint)
        SCMP_REQUIRE(a.out_ld >= a.cols, "scmp_quantize: out_ld < cols");
    return SCMP_OK;
}

// A call the pair launch covers: row groups of a head-symmetric quantizer into codes only,
// dense rows (16-byte aligned, ld = code_ld = cols), no smoothing, row index or given
// ranges, 256 threads of 5 to 16 register-held chunks each: the calls that
// quantize_groups sends to quant_codes_kernel<QOP_MUL, kMaxChunks, kGroupThreads, ...,
// DENSE>. G and npt as that launch takes them.
static bool pair_eligible(const scmp_quant_args &a, int64_t *G_out, int *npt_out) {
    int64_t G, segw, nseg;
    unit_counts(a.rows, a.cols, a.group, a.seg, &G, &segw, &nseg);
    if (nseg != 1 || G > kGroupMaxRows || G * a.cols > (1 << 22) || a.cols < 4) return false;
    if (a.variant != SCMP_Q_HEAD_SYM || a.given_absmax || a.row_index ||
        a.smooth_mode != SCMP_SMOOTH_NONE)
        return false;
    if (!a.code || a.beta16 || a.beta32 || a.sign || a.xint || a.rowsum || a.code_ld % 4 != 0)
        return false;
    if (a.code_kind == SCMP_CODE_THERMO && a.col_class != nullptr) return false;
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    if (cbr % G != 0 || chunk_mode(a) != 0 || a.ld != a.cols || a.code_ld != a.cols)
        return false;
    const int64_t cpr = cdiv(a.cols, 4), ngroups = cdiv(a.rows, G);
    const int64_t ncu = quant_cu_count();
    if (ngroups < 2 * ncu && G * cpr > kBigGroupThreads && G * cpr <= 4 * (int64_t)kBigGroupThreads)
        return false;                                     // the 1024- / 512-thread launches
    const int64_t per = cdiv(G * cpr, kGroupThreads);
    if (per <= 4 || per > kMaxChunks) return false;
    *G_out = G;
    *npt_out = (int)per;
    return true;
}

}  // namespace scmp

using namespace scmp;

extern "C" {

int64_t scmp_quant_workspace_bytes(int64_t rows, int64_t cols, int64_t group, int64_t seg) {
    int64_t G, segw, nseg;
    unit_counts(rows, cols, group, seg, &G, &segw, &nseg);
    int64_t nunits = cdiv(rows, G) * nseg;
    return nunits * (int64_t)(2 * sizeof(uint32_t) + sizeof(QParams)) + 256;
}

int scmp_quantize(const scmp_quant_args *args, hipStream_t stream) {
    SCMP_REQUIRE(args != nullptr, "scmp_quantize: null args");
    scmp_quant_args a = *args;
    {
        const int rc = check_quant_args(a);
        if (rc != SCMP_OK) return rc;
    }
    int64_t G, segw, nseg;
    unit_counts(a.rows, a.cols, a.group, a.seg, &G, &segw, &nseg);
    if (a.variant == SCMP_Q_TENSOR_SYM || a.variant == SCMP_Q_TENSOR_ASYM ||
        a.variant == SCMP_Q_HOST_SYM || a.variant == SCMP_Q_HOST_ASYM) {
        G = a.rows;
        segw = a.cols;
        nseg = 1;
    }
    int64_t nunits = cdiv(a.rows, G) * nseg;
    uint32_t *stats = (uint32_t *)a.workspace;
    uintptr_t pa = ((uintptr_t)(stats + 2 * nunits) + 63) & ~(uintptr_t)63;
    QParams *prm = (QParams *)pa;

    const bool host = a.variant == SCMP_Q_HOST_SYM || a.variant == SCMP_Q_HOST_ASYM;
    const bool tensor = a.variant == SCMP_Q_TENSOR_SYM || a.variant == SCMP_Q_TENSOR_ASYM;
    const bool given = a.given_absmax != nullptr;
    if (given) {
        SCMP_REQUIRE(a.variant == SCMP_Q_GROUP_SYM || a.variant == SCMP_Q_ROW_SYM ||
                     a.variant == SCMP_Q_HEAD_SYM,
                     "scmp_quantize: given_absmax needs a symmetric row-group variant (got %d)",
                     a.variant);
        SCMP_REQUIRE(nseg == 1, "scmp_quantize: given_absmax does not take column segments");
        stats_given_kernel<<<cdiv(nunits, 256), 256, 0, stream>>>(stats, a.given_absmax,
                                                                   nunits);
        SCMP_LAUNCH_CHECK("scmp_quantize/given");
    }
    if (!given && !host && !tensor && nseg == 1 && G <= kGroupMaxRows && G * a.cols <= (1 << 22) &&
        a.cols >= 4 && (!a.code || a.code_ld % 4 == 0))
        return quantize_groups(a, G, stream);
    if (!given && !host && !tensor && nseg > 1 && G == 1 && nseg <= kMaxSegs && segw % 4 == 0 &&
        a.cols <= 4 * kGroupThreads * kMaxChunks && (!a.code || a.code_ld % 4 == 0))
        return quantize_segments(a, segw, nseg, stream);
    if (!host && !given) {
        stats_init_kernel<<<cdiv(2 * nunits, 256), 256, 0, stream>>>(stats, 2 * nunits);
        SCMP_LAUNCH_CHECK("scmp_quantize/init");
        int64_t ntask = a.rows * nseg;
        int64_t blocks = cdiv(ntask, 4);
        if (blocks > 8192) blocks = 8192;
        reduce_kernel<<<blocks, 256, 0, stream>>>(a, G, segw, nseg, stats);
        SCMP_LAUNCH_CHECK("scmp_quantize/reduce");
    }
    finalize_kernel<<<cdiv(nunits, 256), 256, 0, stream>>>(a, nunits, stats, prm);
    SCMP_LAUNCH_CHECK("scmp_quantize/finalize");
    const int64_t cbr = a.code_batch_rows > 0 ? a.code_batch_rows : a.rows;
    int64_t nr = a.code ? (a.rows / cbr) * a.code_rows : a.rows;
    int64_t qblocks = cdiv(nr, 4);
    if (qblocks > 16384) qblocks = 16384;
    quantize_kernel<<<qblocks, 256, 0, stream>>>(a, G, segw, nseg, prm);
    SCMP_LAUNCH_CHECK("scmp_quantize/quantize");
    if (a.scale64 || a.zp64) {
        tensor_out_kernel<<<1, 1, 0, stream>>>(prm, a.scale64, a.zp64);
        SCMP_LAUNCH_CHECK("scmp_quantize/tensor_out");
    }
    return SCMP_OK;
}

int scmp_quantize_pair(const scmp_quant_args *a, const scmp_quant_args *b, hipStream_t stream) {
    SCMP_REQUIRE(a != nullptr && b != nullptr, "scmp_quantize_pair: null args");
    int64_t G1 = 0, G2 = 0;
    int npt1 = 0, npt2 = 0;
    const bool fuse = a->code_kind == SCMP_CODE_THERMO && b->code_kind == SCMP_CODE_Q &&
                      pair_eligible(*a, &G1, &npt1) && pair_eligible(*b, &G2, &npt2);
    if (!fuse) {
        const int rc = scmp_quantize(a, stream);
        return rc != SCMP_OK ? rc : scmp_quantize(b, stream);
    }
    int rc = check_quant_args(*a);
    if (rc != SCMP_OK) return rc;
    rc = check_quant_args(*b);
    if (rc != SCMP_OK) return rc;
    const int64_t n1 = cdiv(a->rows, G1), n2 = cdiv(b->rows, G2);
    SCMP_REQUIRE(n1 + n2 <= (int64_t)INT32_MAX, "scmp_quantize_pair: too many row groups");
    quant_codes_pair_kernel<QOP_MUL, kMaxChunks, kGroupThreads, true>
        <<<(unsigned)(n1 + n2), kGroupThreads, 0, stream>>>(
            *a, *b, (int)n1, (int)G1, (int)cdiv(a->cols, 4), npt1, (int)G2,
            (int)cdiv(b->cols, 4), npt2);
    SCMP_LAUNCH_CHECK("scmp_quantize_pair");
    return SCMP_OK;
}

}  // extern "C"
