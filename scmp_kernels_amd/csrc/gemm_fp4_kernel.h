// SC GEMM kernel on the gfx950 matrix cores with FP4 (e2m1) operands:
// v_mfma_f32_32x32x64_f8f6f4 (cbsz = blgp = 4), twice the int8 rate on MI355X.
//
// Same product as the int8 kernel (gemm_mfma.hip): I[n,m] = sum_d sum_{j' < JPF}
// thermo(code_a)[j'] * lut[class(d)][code_b][j']. Every operand value is a small integer
// that e2m1 represents exactly: the A side is 0 or +-1.0 (nibbles 0x0, 0x2, 0xA), the B
// side an interval count 0..4 or 6 (0x0 0x2 0x4 0x5 0x6 0x7, sign bit 0x8). Products and
// every partial sum are integers of magnitude <= 256 * D <= 2^24 (the host limits D to
// 65536), so the fp32 accumulation is exact and (int)acc == I.
//
// One MFMA covers K = 64 intervals (lane half h: 32 nibbles = 4 dwords). Layout of one
// JPF-nibble table row: dword u (JPF/8 of them), nibble b holds interval j' = (JPF/8)*b + u;
// k-step t, lane half h holds dwords u = 8t + 4h + w. JPF = 32 puts two inner dimensions in
// one k-step (half h takes d = 2p + h); smaller tables are padded to 32. Both operands are
// rows of tables in LDS selected by a code byte: the A thermometer table (row = THERMO
// code) and the stream table (row = B code), so the inner loop is LDS reads and MFMAs.
//
// This header holds the kernel template; gemm_fp4_jp{32,64,128,256}.hip instantiate it
// for one table width each (separate translation units compile in parallel).
#pragma once

#include "gemm_common.h"

namespace scmp {

__device__ __forceinline__ v16f mfma_fp4(v4i a, v4i b, v16f c) {
    v8i A = {a.x, a.y, a.z, a.w, 0, 0, 0, 0};
    v8i B = {b.x, b.y, b.z, b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B, c, 4, 4, 0, 0, 0, 0);
}

// Where the stream tables live: one table in LDS, every class table in LDS (per-d
// classes, when they fit), or per-class tables read from global memory.
enum { LUT_LDS = 0, LUT_LDS_CLASSES = 1, LUT_GLOBAL = 2 };

// floats of the per-wave epilogue staging area: one 32 x 32 block, rows padded to 33
constexpr int kStageFloats = 32 * 33;

template <int JPF>
struct Fp4Geom {
    static constexpr int ROWB = JPF / 2;                         // bytes per table row
    static constexpr int KS = JPF >= 64 ? JPF / 64 : 1;          // MFMA k-steps per d
    static constexpr int UPG = JPF == 32 ? 4 : 8;                // k-step units per 8 codes
    // odd number of 16-byte chunks between LDS rows: spreads rows over the bank groups
    static constexpr int LS = 16 * ((ROWB / 16) | 1);
    static constexpr int TAB = 256 * LS;                          // one table in LDS
};

template <int JPF, int BA, int BB>
struct Fp4Frag {
    v4i a[BA][Fp4Geom<JPF>::KS];
    v4i b[BB][Fp4Geom<JPF>::KS];
};

// The kernel reads both operands from tables indexed by a code byte:
//   A: thermometer table T[code][j'] = sign(code) if j' < j(code) else 0 (built in LDS by
//      the prologue, rows = THERMO code byte: bipolar sign bit | j, unipolar j);
//   B: the stream table lut[class][code_b][j'].
// Each k-step unit (one d, or two d for JPF = 32) is loaded one unit ahead into the other
// of two fragment sets, so the LDS reads of unit u+1 overlap the MFMAs of unit u.
// Interleave one unit's MFMAs with the next unit's LDS reads and address arithmetic:
// per MFMA one DS read (while any remain) and NV VALU instructions.
template <int NM, int NDS, int NV>
__device__ __forceinline__ void interleave_unit() {
#pragma unroll
    for (int k = 0; k < NM; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
        if (k < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);         // VALU
    }
}

template <int JPF, int BA, int BB, int WA, int WB, int LUTSRC, bool CHUNKED, bool SCHED>
__global__ void __launch_bounds__(64 * WA * WB)
sc_gemm_fp4_kernel(GemmP P) {
    using G = Fp4Geom<JPF>;
    constexpr int NT = 64 * WA * WB;
    constexpr int ROWB = G::ROWB, KS = G::KS, UPG = G::UPG, LS = G::LS, TAB = G::TAB;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t *sA = smem;            // thermometer table
    uint8_t *sB = smem + TAB;      // stream table(s) (LUT_LDS, LUT_LDS_CLASSES)
    const uint8_t *glut = (const uint8_t *)P.lut;

    const int tid = threadIdx.x;
    {
        constexpr int U = JPF / 8;                 // dwords per row
        for (int e = tid; e < 256 * U; e += NT) {
            const int row = e / U, u = e - row * U;
            const int j = P.bipolar ? (row & 0x7f) : row;
            const uint32_t one = (P.bipolar && (row & 0x80)) ? 0xAu : 0x2u;
            uint32_t w = 0;
#pragma unroll
            for (int b = 0; b < 8; ++b)
                if (U * b + u < j) w |= one << (4 * b);
            *(uint32_t *)(sA + row * LS + 4 * u) = w;
        }
        if (LUTSRC != LUT_GLOBAL) {
            constexpr int CH = ROWB / 16;         // 16-byte chunks per row
            const int rows = (LUTSRC == LUT_LDS_CLASSES ? P.nclass : 1) * 256;
            const v4i *src = (const v4i *)glut;
            for (int e = tid; e < rows * CH; e += NT) {
                const int row = e / CH, col = e - row * CH;
                *(v4i *)(sB + row * LS + 16 * col) = src[e];
            }
        }
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, li = lane & 31;
    const int wa = wave % WA, wb = wave / WA;
    const int ta = blockIdx.x % P.tilesA, tb = blockIdx.x / P.tilesA;
    const int batch = blockIdx.z;
    const int a0 = (ta * WA + wa) * (BA * 32);
    const int b0 = (tb * WB + wb) * (BB * 32);
    const int D = P.D;
    const int ngroups = (D + 7) / 8;

    const uint8_t *pa[BA];
    const uint8_t *pb[BB];
#pragma unroll
    for (int i = 0; i < BA; ++i) pa[i] = P.ca + batch * P.bsa + (int64_t)(a0 + 32 * i + li) * P.lda;
#pragma unroll
    for (int c = 0; c < BB; ++c) pb[c] = P.cb + batch * P.bsb + (int64_t)(b0 + 32 * c + li) * P.ldb;

    v16f acc[BA][BB];
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int c = 0; c < BB; ++c) acc[i][c] = (v16f){0.0f};
    float yac[CHUNKED ? BA : 1][CHUNKED ? BB : 1][16];
    if (CHUNKED) {
#pragma unroll
        for (int i = 0; i < (CHUNKED ? BA : 1); ++i)
#pragma unroll
            for (int c = 0; c < (CHUNKED ? BB : 1); ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r) yac[i][c][r] = 0.0f;
    }
    const int chunk = P.chunk > 0 ? P.chunk : D;
    int kchunk = 0;

    // fp32 sum over inner-dimension chunks, in chunk order (sc/kernels.py:1333-1381)
    auto flush_chunk = [&](int dlast) __attribute__((always_inline)) {
        const bool end_chunk = ((dlast + 1) % chunk == 0) || (dlast + 1 >= D);
        if (!(end_chunk && dlast < D)) return;
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
                    float raw = __fmul_rn(acc[i][c][r], cc);
                    float term = __fmul_rn(raw, __fmul_rn(san, sbm));
                    yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r] =
                        __fadd_rn(yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r], term);
                    acc[i][c][r] = 0.0f;
                }
        }
        ++kchunk;
    };

    // codes of the current group of 8 d (ca8 / cb8) and of the next one (na / nb)
    uint64_t ca8[BA], cb8[BB];
    uint2 na[BA], nb[BB];
#pragma unroll
    for (int i = 0; i < BA; ++i) {
        const uint2 v = *(const uint2 *)(pa[i]);
        ca8[i] = ((uint64_t)v.y << 32) | v.x;
    }
#pragma unroll
    for (int c = 0; c < BB; ++c) {
        const uint2 v = *(const uint2 *)(pb[c]);
        cb8[c] = ((uint64_t)v.y << 32) | v.x;
    }
    {
        const int g1 = ngroups > 1 ? 1 : 0;
#pragma unroll
        for (int i = 0; i < BA; ++i) na[i] = *(const uint2 *)(pa[i] + 8 * g1);
#pragma unroll
        for (int c = 0; c < BB; ++c) nb[c] = *(const uint2 *)(pb[c] + 8 * g1);
    }

    // load unit `unit` (of the group whose first d is dg) into F
    auto stage = [&](Fp4Frag<JPF, BA, BB> &F, int unit, int dg)
        __attribute__((always_inline)) {
        const int sh = JPF == 32 ? 8 * (2 * unit + h) : 8 * unit;
#pragma unroll
        for (int i = 0; i < BA; ++i) {
            const int code = (int)((ca8[i] >> sh) & 0xff);
            const uint8_t *p = sA + code * LS + (JPF == 32 ? 0 : 16 * h);
#pragma unroll
            for (int t = 0; t < KS; ++t) F.a[i][t] = *(const v4i *)(p + 32 * t);
        }
        const uint8_t *base = sB;
        if (LUTSRC != LUT_LDS) {
            const int d = dg + (JPF == 32 ? 2 * unit + h : unit);
            const int cls = d < D ? P.d_class[d] : 0;
            base = LUTSRC == LUT_GLOBAL ? glut + (int64_t)cls * 256 * ROWB : sB + cls * TAB;
        }
#pragma unroll
        for (int c = 0; c < BB; ++c) {
            const int code = (int)((cb8[c] >> sh) & 0xff);
            const uint8_t *p = base + code * (LUTSRC == LUT_GLOBAL ? ROWB : LS) +
                               (JPF == 32 ? 0 : 16 * h);
#pragma unroll
            for (int t = 0; t < KS; ++t) F.b[c][t] = *(const v4i *)(p + 32 * t);
        }
    };
    auto mma = [&](const Fp4Frag<JPF, BA, BB> &F) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < KS; ++t)
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int c = 0; c < BB; ++c) acc[i][c] = mfma_fp4(F.a[i][t], F.b[c][t], acc[i][c]);
    };
    auto after = [&](int unit, int dg) __attribute__((always_inline)) {
        if (CHUNKED) {
            const int dlast = dg + (JPF == 32 ? 2 * unit + 1 : unit);
            if (dg + (JPF == 32 ? 2 * unit : unit) < D) flush_chunk(dlast < D ? dlast : D - 1);
        }
    };

    Fp4Frag<JPF, BA, BB> F0, F1;
    stage(F0, 0, 0);
    for (int g = 0; g < ngroups; ++g) {
        const int dg = 8 * g;
#pragma unroll
        for (int uu = 0; uu < UPG; uu += 2) {
            stage(F1, uu + 1, dg);
            mma(F0);
            if (SCHED) interleave_unit<BA * BB * KS, (BA + BB) * KS, 1>();
            after(uu, dg);
            if (uu + 2 < UPG) {
                stage(F0, uu + 2, dg);
            } else {
                // rotate to the next group; the group after it is fetched now (clamped to
                // the last group, whose codes are then loaded but never used)
#pragma unroll
                for (int i = 0; i < BA; ++i) ca8[i] = ((uint64_t)na[i].y << 32) | na[i].x;
#pragma unroll
                for (int c = 0; c < BB; ++c) cb8[c] = ((uint64_t)nb[c].y << 32) | nb[c].x;
                const int g2 = g + 2 < ngroups ? g + 2 : ngroups - 1;
#pragma unroll
                for (int i = 0; i < BA; ++i) na[i] = *(const uint2 *)(pa[i] + 8 * g2);
#pragma unroll
                for (int c = 0; c < BB; ++c) nb[c] = *(const uint2 *)(pb[c] + 8 * g2);
                stage(F0, 0, dg + 8);
            }
            mma(F1);
            if (SCHED) interleave_unit<BA * BB * KS, (BA + BB) * KS, 1>();
            after(uu + 1, dg);
        }
    }

    if (CHUNKED) {
        // the chunked fp32 sums are the final values
#pragma unroll
        for (int c = 0; c < BB; ++c) {
            const int m = b0 + 32 * c + li;
            if (m >= P.M) continue;
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = a0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (n >= P.N) continue;
                    P.y[batch * P.bsy + (int64_t)n * P.ldy + m] =
                        yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r];
                }
        }
        return;
    }

    // Fused epilogue. Each 32 x 32 accumulator block is staged through a per-wave LDS
    // area (the tables are dead by now), then read back row-wise: lanes 0-31 / 32-63 take
    // 32 consecutive m of rows 2k / 2k+1, so the fp32 stores are coalesced and the
    // accumulator registers are only ever read by LDS stores.
    __syncthreads();
    float *stg = (float *)smem + wave * kStageFloats;
    const int ecol = lane & 31, ehalf = lane >> 5;
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int c = 0; c < BB; ++c) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                stg[(8 * (r >> 2) + 4 * h + (r & 3)) * 33 + li] = acc[i][c][r];
            __syncthreads();
            const int m = b0 + 32 * c + ecol;
#pragma unroll 2
            for (int rr = ehalf; rr < 32; rr += 2) {
                const int n = a0 + 32 * i + rr;
                const float v = stg[rr * 33 + ecol];
                if (n < P.N && m < P.M) {
                    const int64_t o = batch * P.bsy + (int64_t)n * P.ldy + m;
                    if (P.epi.kind == SCMP_EPI_INT) P.iout[o] = (int32_t)v;
                    else P.y[o] = epilogue_value(P.epi, v, n, m, batch);
                }
            }
            __syncthreads();
        }
}

// Largest LDS request of one workgroup (gfx950: 160 KiB per CU).
constexpr int kFp4MaxLds = 160 * 1024;

template <int JPF, int BA, int BB, int WA, int WB, int LUTSRC, bool CHUNKED, bool SCHED>
static int launch_fp4_t(const GemmP &P0, int64_t batch, hipStream_t stream) {
    using G = Fp4Geom<JPF>;
    GemmP P = P0;
    const int tileA = WA * BA * 32, tileB = WB * BB * 32;
    P.tilesA = (int)cdiv(P.N, tileA);
    const int64_t tilesB = cdiv(P.M, tileB);
    const int ntab = LUTSRC == LUT_LDS ? 1 : LUTSRC == LUT_LDS_CLASSES ? P.nclass : 0;
    size_t lds = (size_t)G::TAB * (1 + ntab);
    const size_t stage = CHUNKED ? 0 : (size_t)WA * WB * kStageFloats * sizeof(float);
    if (lds < stage) lds = stage;
    auto kern = sc_gemm_fp4_kernel<JPF, BA, BB, WA, WB, LUTSRC, CHUNKED, SCHED>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void *)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) {
            set_error("scmp_sc_gemm(mfma fp4): %zu bytes of LDS refused: %s", lds,
                      hipGetErrorString(e));
            return SCMP_E_LAUNCH;
        }
    }
    dim3 grid((unsigned)(P.tilesA * tilesB), 1, (unsigned)batch);
    kern<<<grid, 64 * WA * WB, lds, stream>>>(P);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma fp4)");
    return SCMP_OK;
}

// Tiles (A rows x B rows per workgroup):
//  non-chunked: 256 x 256, each wave 128 x 128 (4 x 4 blocks of 32 x 32), MFMA / LDS-read
//               interleaving enforced, epilogue fused;
//  chunked:     128 x 128, each wave 64 x 64 (2 x 2 blocks, fp32 chunk sums in registers).
template <int JPF, int LUTSRC>
static int launch_fp4_jp(const GemmP &P, int64_t batch, bool chunked, hipStream_t s) {
    if (chunked) return launch_fp4_t<JPF, 2, 2, 2, 2, LUTSRC, true, false>(P, batch, s);
    return launch_fp4_t<JPF, 4, 4, 2, 2, LUTSRC, false, true>(P, batch, s);
}

// Stream tables: one shared table in LDS; every class table in LDS when they fit;
// otherwise per-class rows read from global memory.
template <int JPF>
int gemm_fp4_launch_jpf(const GemmP &P, int64_t batch, bool chunked, hipStream_t s) {
    if (P.d_class == nullptr) return launch_fp4_jp<JPF, LUT_LDS>(P, batch, chunked, s);
    if (P.nclass > 0 && (int64_t)Fp4Geom<JPF>::TAB * (1 + P.nclass) <= kFp4MaxLds)
        return launch_fp4_jp<JPF, LUT_LDS_CLASSES>(P, batch, chunked, s);
    return launch_fp4_jp<JPF, LUT_GLOBAL>(P, batch, chunked, s);
}

}  // namespace scmp
