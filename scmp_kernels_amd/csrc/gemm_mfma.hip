// SC GEMM on the gfx950 matrix cores (v_mfma_i32_32x32x32_i8).
//
// The reference's enable-signal matmul (scmp_kernels/sc/kernels.py:176-252) computes
//   I[n,m] = sum_d s_a s_b C[d, K[d, beta_a], beta_b],  C[d,k,v] = #{i < k : r_b[d,i] < v}
// i.e. a thermometer code of length K_a ANDed with the B-side compare stream, popcounted.
// Positions i are grouped into "intervals" between consecutive attainable K_a values
// (kappa_0 < ... < kappa_J); then
//   I[n,m] = sum_d sum_{j' < J} [j' < j_a] * s_a * s_b * Dlt[d][q_b][j']
// where j_a = index of K_a and Dlt[..][j'] = #{i in interval j' : r_b[i] < beta(q_b)}
// (0..3 for the default configs). That is an int8 GEMM with K = D * JP:
//   A operand: signed thermometer of length j_a (built in registers, no memory),
//   B operand: one LUT row per (m, d) (256 rows x JP bytes per table class, in LDS),
// accumulated exactly in int32 by the MFMA. JP = 128 for the 8-bit bipolar grid, half
// the 256 stream positions of the reference's L = 256 (the 127 attainable boundaries).
//
// Byte layout inside one JP-byte row (both operands): dword u, byte b holds interval
// j' = (JP/4)*b + u. With j_a = (JP/4)*qq + rr the A dword u is PART if u < rr else FULL,
// where FULL has the sign byte in bytes b < qq and PART additionally in byte qq: two VALU
// ops (v_cmp + v_cndmask) per dword. For one k-step of 32 (two 16-byte lane halves h)
// lane half h holds dwords u = 8t + 4h + w, w = 0..3, of every row. JP = 16 packs two d
// per k-step instead (half h takes d = 2p + h).
//
// Waves are independent (no inter-wave data sharing besides the read-only LUT in LDS).
#include "common.h"

namespace scmp {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef char v16c __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));

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
    int tilesA;
};

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v16c, a),
                                                 __builtin_bit_cast(v16c, b), c, 0, 0, 0);
}

// (FULL, PART) dword pair of a thermometer code (see file comment).
__device__ __forceinline__ uint2 fp_of_code(int code, int JP, int bipolar) {
    int j = bipolar ? (code & 0x7f) : code;
    uint32_t spat = (bipolar && (code & 0x80)) ? 0xffffffffu : 0x01010101u;
    int U = JP / 4;
    int qq = j / U;
    uint32_t full = qq >= 4 ? 0xffffffffu : (uint32_t)((1ull << (8 * qq)) - 1ull);
    full &= spat;
    uint32_t part = qq >= 4 ? full : (full | (spat & (0xffu << (8 * qq))));
    return make_uint2(full, part);
}

template <int JP, int BA, int BB, int WA, int WB, bool PERCLASS, bool CHUNKED>
__global__ void __launch_bounds__(64 * WA * WB)
sc_gemm_mfma_kernel(GemmP P) {
    constexpr int NT = 64 * WA * WB;
    constexpr int U = JP / 4;                  // dwords per row
    constexpr int KSTEPS = JP >= 32 ? JP / 32 : 1;
    __shared__ uint2 fptab[256];
    __shared__ __attribute__((aligned(16))) int8_t slut[PERCLASS ? 16 : 256 * JP];

    const int tid = threadIdx.x;
    for (int e = tid; e < 256; e += NT) fptab[e] = fp_of_code(e, JP, P.bipolar);
    if (!PERCLASS) {
        const v4i *src = (const v4i *)P.lut;
        v4i *dst = (v4i *)slut;
        for (int e = tid; e < 256 * JP / 16; e += NT) dst[e] = src[e];
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, li = lane & 31;
    const int wa = wave % WA, wb = wave / WA;
    const int ta = blockIdx.x % P.tilesA, tb = blockIdx.x / P.tilesA;
    const int batch = blockIdx.z;
    const int a0 = (ta * WA + wa) * (BA * 32);
    const int b0 = (tb * WB + wb) * (BB * 32);

    const uint8_t *pa[BA];
    const uint8_t *pb[BB];
#pragma unroll
    for (int i = 0; i < BA; ++i) pa[i] = P.ca + batch * P.bsa + (int64_t)(a0 + 32 * i + li) * P.lda;
#pragma unroll
    for (int c = 0; c < BB; ++c) pb[c] = P.cb + batch * P.bsb + (int64_t)(b0 + 32 * c + li) * P.ldb;

    v16i acc[BA][BB];
    float yac[CHUNKED ? BA : 1][CHUNKED ? BB : 1][16];
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int c = 0; c < BB; ++c) acc[i][c] = (v16i){0};
    if (CHUNKED) {
#pragma unroll
        for (int i = 0; i < (CHUNKED ? BA : 1); ++i)
#pragma unroll
            for (int c = 0; c < (CHUNKED ? BB : 1); ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r) yac[i][c][r] = 0.0f;
    }

    const int D = P.D;
    const int ngroups = (D + 7) / 8;
    const int chunk = P.chunk > 0 ? P.chunk : D;
    int kchunk = 0;

    uint2 na[BA], nb[BB];
#pragma unroll
    for (int i = 0; i < BA; ++i) na[i] = *(const uint2 *)(pa[i]);
#pragma unroll
    for (int c = 0; c < BB; ++c) nb[c] = *(const uint2 *)(pb[c]);

    for (int g = 0; g < ngroups; ++g) {
        uint64_t ca8[BA], cb8[BB];
#pragma unroll
        for (int i = 0; i < BA; ++i) ca8[i] = ((uint64_t)na[i].y << 32) | na[i].x;
#pragma unroll
        for (int c = 0; c < BB; ++c) cb8[c] = ((uint64_t)nb[c].y << 32) | nb[c].x;
        if (g + 1 < ngroups) {
#pragma unroll
            for (int i = 0; i < BA; ++i) na[i] = *(const uint2 *)(pa[i] + 8 * (g + 1));
#pragma unroll
            for (int c = 0; c < BB; ++c) nb[c] = *(const uint2 *)(pb[c] + 8 * (g + 1));
        }
        const int dbase = 8 * g;
        constexpr int DSTEP = JP == 16 ? 2 : 1;
#pragma unroll 1
        for (int dd = 0; dd < 8; dd += DSTEP) {
            // JP == 16: this lane half works on d = dbase + dd + h
            const int sh = JP == 16 ? 8 * (dd + h) : 8 * dd;
            uint32_t full[BA], part[BA];
            int rr[BA];
#pragma unroll
            for (int i = 0; i < BA; ++i) {
                const int code = (int)((ca8[i] >> sh) & 0xff);
                const uint2 fp = fptab[code];
                full[i] = fp.x;
                part[i] = fp.y;
                rr[i] = JP == 16 ? (code & 3) : ((code & (U - 1)) - 4 * h);
            }
            const int8_t *lp[BB];
#pragma unroll
            for (int c = 0; c < BB; ++c) {
                const int code = (int)((cb8[c] >> sh) & 0xff);
                const int8_t *base;
                if (PERCLASS) {
                    const int dcur = dbase + dd + (JP == 16 ? h : 0);
                    const int cls = (P.d_class && dcur < D) ? P.d_class[dcur] : 0;
                    base = P.lut + (int64_t)cls * 256 * JP;
                } else {
                    base = slut;
                }
                lp[c] = base + code * JP + (JP == 16 ? 0 : 16 * h);
            }
#pragma unroll
            for (int t = 0; t < KSTEPS; ++t) {
                v4i bf[BB];
#pragma unroll
                for (int c = 0; c < BB; ++c) bf[c] = *(const v4i *)(lp[c] + 32 * t);
#pragma unroll
                for (int i = 0; i < BA; ++i) {
                    v4i af;
                    af.x = (8 * t + 0 < rr[i]) ? part[i] : full[i];
                    af.y = (8 * t + 1 < rr[i]) ? part[i] : full[i];
                    af.z = (8 * t + 2 < rr[i]) ? part[i] : full[i];
                    af.w = (8 * t + 3 < rr[i]) ? part[i] : full[i];
#pragma unroll
                    for (int c = 0; c < BB; ++c) acc[i][c] = mfma_i8(af, bf[c], acc[i][c]);
                }
            }
            if (CHUNKED) {
                // flush at the end of every inner-dimension chunk, in chunk order
                const int dlast = dbase + dd + DSTEP - 1;
                const bool end_chunk = ((dlast + 1) % chunk == 0) || (dlast + 1 >= D);
                if (end_chunk && dlast < D + DSTEP - 1) {
                    const float cc = P.epi.c;
                    const float *sa = P.epi.sa + (int64_t)kchunk * P.epi.sa_chunk_stride;
                    const float *sb = P.epi.sb + (int64_t)kchunk * P.epi.sb_chunk_stride;
#pragma unroll
                    for (int c = 0; c < BB; ++c) {
                        const int m = b0 + 32 * c + li;
                        const float sbm = m < P.M ? sb[m] : 0.0f;
#pragma unroll
                        for (int i = 0; i < BA; ++i)
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const int n = a0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                                const float san = n < P.N ? sa[n] : 0.0f;
                                float raw = __fmul_rn((float)acc[i][c][r], cc);
                                float term = __fmul_rn(raw, __fmul_rn(san, sbm));
                                yac[i][c][r] = __fadd_rn(yac[i][c][r], term);
                                acc[i][c][r] = 0;
                            }
                    }
                    ++kchunk;
                }
            }
        }
    }

    // ---------------- store ----------------
    // Non-chunked kernels store the exact int32 I; the fp32 epilogue runs as a separate
    // elementwise pass (epilogue_kernel, in place over the same buffer). Fusing it here
    // makes the register allocator move all accumulators out of the AGPRs and spill.
#pragma unroll
    for (int c = 0; c < BB; ++c) {
        const int m = b0 + 32 * c + li;
        if (m >= P.M) continue;
#pragma unroll
        for (int i = 0; i < BA; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = a0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                if (n >= P.N) continue;
                const int64_t o = batch * P.bsy + (int64_t)n * P.ldy + m;
                if (CHUNKED) {
                    P.y[o] = yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r];
                    continue;
                }
                P.iout[o] = acc[i][c][r];
            }
        }
    }
}

// fp32 epilogues of the reference paths, applied to the int32 accumulator in place.
__global__ void epilogue_kernel(const int32_t *iin, float *y, int N, int M, int64_t ldy,
                                int64_t bsy, scmp_epilogue E) {
    const int batch = blockIdx.z;
    for (int n = blockIdx.y; n < N; n += gridDim.y)
    for (int m = blockIdx.x * blockDim.x + threadIdx.x; m < M; m += gridDim.x * blockDim.x) {
        const int64_t o = batch * bsy + (int64_t)n * ldy + m;
        const float I = (float)iin[o];
        float out;
        switch (E.kind) {
        case SCMP_EPI_ROWCOL: {
            // fl(fl(I*c) * fl(sa*sb)): sc/kernels.py:248 then :1707 / :1271 / :1894
            float raw = __fmul_rn(I, E.c);
            float s = __fmul_rn(E.sa[batch * E.sa_batch_stride + n],
                                E.sb[batch * E.sb_batch_stride + m]);
            out = __fmul_rn(raw, s);
            break;
        }
        case SCMP_EPI_SCALAR:  // sc/kernels.py:1204 (scale product is a float64 value)
            out = __fmul_rn(__fmul_rn(I, E.c), E.s[0]);
            break;
        case SCMP_EPI_HEAD:    // sc/kernels.py:430-432
            out = __fmul_rn(I, __fmul_rn(E.c, E.s[batch]));
            break;
        case SCMP_EPI_ZP_ROWCOL: {  // sc/kernels.py:1699-1707
            const int64_t na_ = batch * E.sa_batch_stride + n;
            const int64_t mb_ = batch * E.sb_batch_stride + m;
            float raw = __fmul_rn(I, E.c);
            float za = E.za[na_], zb = E.zb[mb_];
            float t1 = __fmul_rn(-zb, E.suma[na_]);
            float t2 = __fmul_rn(za, E.sumb[mb_]);
            float t3 = __fmul_rn(__fmul_rn(E.dfloat, za), zb);
            float corr = __fadd_rn(__fsub_rn(t1, t2), t3);
            raw = __fadd_rn(raw, corr);
            out = __fmul_rn(raw, __fmul_rn(E.sa[na_], E.sb[mb_]));
            break;
        }
        default: {  // SCMP_EPI_ZP_SCALAR, sc/kernels.py:1198-1204
            float raw = __fmul_rn(I, E.c);
            float t1 = __fmul_rn(-E.zb[0], E.suma[batch * E.sa_batch_stride + n]);
            float t2 = __fmul_rn(E.za[0], E.sumb[batch * E.sb_batch_stride + m]);
            float corr = __fadd_rn(__fsub_rn(t1, t2), E.t3[0]);
            raw = __fadd_rn(raw, corr);
            out = __fmul_rn(raw, E.s[0]);
            break;
        }
        }
        y[o] = out;
    }
}

int run_epilogue(const int32_t *iin, float *y, int64_t N, int64_t M, int64_t batch,
                 int64_t ldy, int64_t bsy, const scmp_epilogue &E, hipStream_t stream) {
    int64_t bx = cdiv(M, 256);
    if (bx > 64) bx = 64;
    dim3 grid((unsigned)bx, (unsigned)(N < 32768 ? N : 32768), (unsigned)batch);
    epilogue_kernel<<<grid, 256, 0, stream>>>(iin, y, (int)N, (int)M, ldy, bsy, E);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(epilogue)");
    return SCMP_OK;
}

template <int JP, int BA, int BB, int WA, int WB, bool PERCLASS, bool CHUNKED>
static int launch_t(const GemmP &P0, int64_t batch, hipStream_t stream) {
    GemmP P = P0;
    const int tileA = WA * BA * 32, tileB = WB * BB * 32;
    P.tilesA = (int)cdiv(P.N, tileA);
    const int64_t tilesB = cdiv(P.M, tileB);
    dim3 grid((unsigned)(P.tilesA * tilesB), 1, (unsigned)batch);
    sc_gemm_mfma_kernel<JP, BA, BB, WA, WB, PERCLASS, CHUNKED><<<grid, 64 * WA * WB, 0, stream>>>(P);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma)");
    return SCMP_OK;
}

// Tile presets: rows of A (thermometer side) x rows of B (LUT side) per workgroup.
//  0: 256 x 256, each wave 256 x 64 (8 x 2 blocks of 32x32, 256 accumulator registers)
//  1: 256 x 128, each wave 128 x 64 (4 x 2 blocks)
//  chunked epilogue: 128 x 128, each wave 64 x 64 (2 x 2 blocks, fp32 sums in registers)
template <int JP, bool PERCLASS>
static int launch_jp(const GemmP &P, int64_t batch, int tile, bool chunked, hipStream_t s) {
    if (chunked) return launch_t<JP, 2, 2, 2, 2, PERCLASS, true>(P, batch, s);
    if (tile == 1) return launch_t<JP, 4, 2, 2, 2, PERCLASS, false>(P, batch, s);
    return launch_t<JP, 8, 2, 1, 4, PERCLASS, false>(P, batch, s);
}

template <bool PERCLASS>
static int launch_pc(const GemmP &P, int64_t batch, int JP, int tile, bool chunked,
                     hipStream_t s) {
    switch (JP) {
    case 16: return launch_jp<16, PERCLASS>(P, batch, tile, chunked, s);
    case 32: return launch_jp<32, PERCLASS>(P, batch, tile, chunked, s);
    case 64: return launch_jp<64, PERCLASS>(P, batch, tile, chunked, s);
    case 128: return launch_jp<128, PERCLASS>(P, batch, tile, chunked, s);
    default: return launch_jp<256, PERCLASS>(P, batch, tile, chunked, s);
    }
}

int gemm_valu_launch(const scmp_gemm_args &a, hipStream_t stream);  // gemm_valu.hip

}  // namespace scmp

using namespace scmp;

extern "C" int scmp_sc_gemm(const scmp_gemm_args *args, hipStream_t stream) {
    SCMP_REQUIRE(args != nullptr, "scmp_sc_gemm: null args");
    const scmp_gemm_args &a = *args;
    SCMP_REQUIRE(a.ca && a.cb && a.lut, "scmp_sc_gemm: null code/lut pointer");
    SCMP_REQUIRE(a.N > 0 && a.M > 0 && a.D > 0 && a.batch > 0,
                 "scmp_sc_gemm: empty problem N=%lld M=%lld D=%lld batch=%lld",
                 (long long)a.N, (long long)a.M, (long long)a.D, (long long)a.batch);
    SCMP_REQUIRE(a.N < (1LL << 30) && a.M < (1LL << 30) && a.D < (1LL << 24) &&
                     a.batch < 65536,
                 "scmp_sc_gemm: dimensions too large");
    SCMP_REQUIRE(a.JP == 16 || a.JP == 32 || a.JP == 64 || a.JP == 128 || a.JP == 256,
                 "scmp_sc_gemm: JP=%d must be 16, 32, 64, 128 or 256", a.JP);
    SCMP_REQUIRE(a.lda % 16 == 0 && a.ldb % 16 == 0 && a.lda >= cdiv(a.D, 16) * 16 &&
                     a.ldb >= cdiv(a.D, 16) * 16,
                 "scmp_sc_gemm: code row strides (%lld, %lld) must be multiples of 16 and "
                 ">= D rounded up to 16", (long long)a.lda, (long long)a.ldb);
    SCMP_REQUIRE(a.epi.kind >= SCMP_EPI_INT && a.epi.kind <= SCMP_EPI_ZP_SCALAR,
                 "scmp_sc_gemm: unknown epilogue kind %d", a.epi.kind);
    SCMP_REQUIRE(a.epi.kind == SCMP_EPI_INT ? a.iout != nullptr : a.y != nullptr,
                 "scmp_sc_gemm: missing output buffer");
    SCMP_REQUIRE(a.ldy >= a.M, "scmp_sc_gemm: ldy < M");
    const bool chunked = a.chunk > 0 && a.chunk < a.D;
    SCMP_REQUIRE(!chunked || a.epi.kind == SCMP_EPI_ROWCOL,
                 "scmp_sc_gemm: chunked accumulation needs the ROWCOL epilogue");
    SCMP_REQUIRE(!chunked || a.impl == SCMP_GEMM_MFMA,
                 "scmp_sc_gemm: chunked accumulation is implemented by the MFMA kernel");
    if (a.impl == SCMP_GEMM_VALU) return gemm_valu_launch(a, stream);
    SCMP_REQUIRE(a.impl == SCMP_GEMM_MFMA, "scmp_sc_gemm: unknown impl %d", a.impl);
    GemmP P;
    P.ca = a.ca; P.lda = a.lda; P.bsa = a.bsa;
    P.cb = a.cb; P.ldb = a.ldb; P.bsb = a.bsb;
    P.N = (int)a.N; P.M = (int)a.M; P.D = (int)a.D;
    P.chunk = chunked ? (int)a.chunk : 0;
    P.lut = a.lut; P.d_class = a.d_class; P.bipolar = a.bipolar;
    P.epi = a.epi; P.y = a.y; P.ldy = a.ldy; P.bsy = a.bsy;
    // non-chunked: int32 I goes to iout, or into the fp32 output buffer itself (the
    // epilogue pass then converts it in place)
    P.iout = a.epi.kind == SCMP_EPI_INT ? a.iout : (int32_t *)a.y;
    P.tilesA = 0;
    const bool perclass = a.d_class != nullptr;
    int rc = perclass ? launch_pc<true>(P, a.batch, a.JP, a.tile, chunked, stream)
                      : launch_pc<false>(P, a.batch, a.JP, a.tile, chunked, stream);
    if (rc != SCMP_OK || chunked || a.epi.kind == SCMP_EPI_INT) return rc;
    return run_epilogue(P.iout, a.y, a.N, a.M, a.batch, a.ldy, a.bsy, a.epi, stream);
}
