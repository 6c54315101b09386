// SC GEMM on the gfx950 matrix cores with FP4 (e2m1) operands:
// v_mfma_f32_32x32x64_f8f6f4 (cbsz = blgp = 4), twice the int8 rate on MI355X.
//
// Same product as the int8 kernel (gemm_mfma.hip): I[n,m] = sum_d sum_{j' < JPF}
// thermo(code_a)[j'] * lut[class(d)][code_b][j']. Every operand value is a small integer
// that e2m1 represents exactly: the A side is 0 or +-1.0 (nibbles 0x0, 0x2, 0xA), the B
// side an interval count 0..4 or 6 (0x0 0x2 0x4 0x5 0x6 0x7, sign bit 0x8). Products and
// every partial sum are integers of magnitude <= D * 256 < 2^24, so the fp32 accumulation
// is exact and (int)acc == I.
//
// One MFMA covers K = 64 intervals (lane half h: 32 nibbles = 4 dwords). Layout of one
// JPF-nibble row: dword u (JPF/8 of them), nibble b holds interval j' = (JPF/8)*b + u, so
// with j_a = (JPF/8)*qq + rr the A dword u is PART if u < rr else FULL (the FULL word has
// the sign nibble in nibbles < qq, PART also in nibble qq). K-step t, lane half h holds
// dwords u = 8t + 4h + w. JPF = 32 puts two inner dimensions in one K-step (half h takes
// d = 2p + h); smaller tables are padded to 32.
#include "gemm_common.h"

namespace scmp {

__device__ __forceinline__ v16f mfma_fp4(v4i a, v4i b, v16f c) {
    v8i A = {a.x, a.y, a.z, a.w, 0, 0, 0, 0};
    v8i B = {b.x, b.y, b.z, b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B, c, 4, 4, 0, 0, 0, 0);
}

template <int JPF>
__device__ __forceinline__ void thermo_pair4(int code, bool bipolar, uint32_t &full,
                                             uint32_t &part, int &rr, int h) {
    constexpr int U = JPF / 8;
    const int j = bipolar ? (code & 0x7f) : code;
    const int qq = j / U;                                  // 0..8
    const uint32_t neg = bipolar ? (uint32_t)((int)((uint32_t)code << 24) >> 31) : 0u;
    const uint32_t spat = (neg & 0x88888888u) | 0x22222222u;   // nibbles of -1.0 / +1.0
    const int w = 4 * qq;
    const uint32_t m = qq >= 8 ? 0xffffffffu : ((1u << (w & 31)) - 1u);
    full = m & spat;
    part = qq >= 8 ? full : (full | (spat & (0xfu << (w & 31))));
    rr = JPF == 32 ? (j & 3) : ((j & (U - 1)) - 4 * h);
}

template <int JPF, int BA, int BB, int WA, int WB, bool PERCLASS, bool CHUNKED>
__global__ void __launch_bounds__(64 * WA * WB)
sc_gemm_fp4_kernel(GemmP P) {
    constexpr int NT = 64 * WA * WB;
    constexpr int ROWB = JPF / 2;                          // bytes per LUT row
    constexpr int KSTEPS = JPF >= 64 ? JPF / 64 : 1;
    // odd number of 16-byte chunks between rows: spreads rows over the LDS bank groups
    constexpr int LSTRIDE = 16 * ((ROWB / 16) | 1);
    __shared__ __attribute__((aligned(16))) uint8_t slut[PERCLASS ? 16 : 256 * LSTRIDE];
    const uint8_t *glut = (const uint8_t *)P.lut;

    const int tid = threadIdx.x;
    if (!PERCLASS) {
        const v4i *src = (const v4i *)glut;
        for (int e = tid; e < 256 * ROWB / 16; e += NT) {
            const int row = e / (ROWB / 16), col = e - row * (ROWB / 16);
            *(v4i *)(slut + row * LSTRIDE + 16 * col) = src[e];
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

    const uint8_t *pa[BA];
    const uint8_t *pb[BB];
#pragma unroll
    for (int i = 0; i < BA; ++i) pa[i] = P.ca + batch * P.bsa + (int64_t)(a0 + 32 * i + li) * P.lda;
#pragma unroll
    for (int c = 0; c < BB; ++c) pb[c] = P.cb + batch * P.bsb + (int64_t)(b0 + 32 * c + li) * P.ldb;

    v16f acc[BA][BB];
    float yac[CHUNKED ? BA : 1][CHUNKED ? BB : 1][16];
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int c = 0; c < BB; ++c) acc[i][c] = (v16f){0.0f};
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

    auto flush_chunk = [&](int dlast) {
        // fp32 sum over inner-dimension chunks, in chunk order (sc/kernels.py:1333-1381)
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
        constexpr int DSTEP = JPF == 32 ? 2 : 1;
#pragma unroll 1
        for (int dd = 0; dd < 8; dd += DSTEP) {
            // JPF == 32: this lane half works on d = dbase + dd + h
            const int sh = JPF == 32 ? 8 * (dd + h) : 8 * dd;
            uint32_t full[BA], part[BA];
            int rr[BA];
#pragma unroll
            for (int i = 0; i < BA; ++i)
                thermo_pair4<JPF>((int)((ca8[i] >> sh) & 0xff), P.bipolar, full[i], part[i],
                                  rr[i], h);
            const uint8_t *base;
            if (PERCLASS) {
                const int dcur = dbase + dd + (JPF == 32 ? h : 0);
                const int cls = (P.d_class && dcur < D) ? P.d_class[dcur] : 0;
                base = glut + (int64_t)cls * 256 * ROWB;
            } else {
                base = slut;
            }
            const uint8_t *lp[BB];
#pragma unroll
            for (int c = 0; c < BB; ++c)
                lp[c] = base + (int)((cb8[c] >> sh) & 0xff) * (PERCLASS ? ROWB : LSTRIDE) +
                        (JPF == 32 ? 0 : 16 * h);
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
                    for (int c = 0; c < BB; ++c) acc[i][c] = mfma_fp4(af, bf[c], acc[i][c]);
                }
            }
            if (CHUNKED && dbase + dd < D)
                flush_chunk(dbase + dd + DSTEP - 1 < D ? dbase + dd + DSTEP - 1 : D - 1);
        }
    }

    // store the exact integer accumulator (or the chunked fp32 sums)
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
                P.iout[o] = (int32_t)acc[i][c][r];
            }
        }
    }
}

template <int JPF, int BA, int BB, int WA, int WB, bool PERCLASS, bool CHUNKED>
static int launch_fp4_t(const GemmP &P0, int64_t batch, hipStream_t stream) {
    GemmP P = P0;
    const int tileA = WA * BA * 32, tileB = WB * BB * 32;
    P.tilesA = (int)cdiv(P.N, tileA);
    const int64_t tilesB = cdiv(P.M, tileB);
    dim3 grid((unsigned)(P.tilesA * tilesB), 1, (unsigned)batch);
    sc_gemm_fp4_kernel<JPF, BA, BB, WA, WB, PERCLASS, CHUNKED>
        <<<grid, 64 * WA * WB, 0, stream>>>(P);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma fp4)");
    return SCMP_OK;
}

// Tile presets (A rows x B rows per workgroup):
//  0: 256 x 256, each wave 128 x 128 (4 x 4 blocks)
//  1: 256 x 256, each wave 256 x 64 (8 x 2 blocks)
//  chunked epilogue: 128 x 128, each wave 64 x 64 (2 x 2 blocks, fp32 sums in registers)
template <int JPF, bool PERCLASS>
static int launch_fp4_jp(const GemmP &P, int64_t batch, int tile, bool chunked,
                         hipStream_t s) {
    if (chunked) return launch_fp4_t<JPF, 2, 2, 2, 2, PERCLASS, true>(P, batch, s);
    if (tile == 1) return launch_fp4_t<JPF, 8, 2, 1, 4, PERCLASS, false>(P, batch, s);
    return launch_fp4_t<JPF, 4, 4, 2, 2, PERCLASS, false>(P, batch, s);
}

int gemm_fp4_launch(const GemmP &P, int64_t batch, int JPF, int tile, bool chunked,
                    hipStream_t stream) {
    const bool pc = P.d_class != nullptr;
    switch (JPF) {
    case 32: return pc ? launch_fp4_jp<32, true>(P, batch, tile, chunked, stream)
                       : launch_fp4_jp<32, false>(P, batch, tile, chunked, stream);
    case 64: return pc ? launch_fp4_jp<64, true>(P, batch, tile, chunked, stream)
                       : launch_fp4_jp<64, false>(P, batch, tile, chunked, stream);
    case 128: return pc ? launch_fp4_jp<128, true>(P, batch, tile, chunked, stream)
                        : launch_fp4_jp<128, false>(P, batch, tile, chunked, stream);
    case 256: return pc ? launch_fp4_jp<256, true>(P, batch, tile, chunked, stream)
                        : launch_fp4_jp<256, false>(P, batch, tile, chunked, stream);
    default: set_error("scmp_sc_gemm(fp4): JPF=%d unsupported", JPF); return SCMP_E_ARG;
    }
}

// FP4 table from the int8 stream table: row stride JPF/2 bytes, nibble layout above.
// Counts outside e2m1's integers {0, 1, 2, 3, 4, 6} set *bad.
__global__ void fp4_lut_kernel(const int8_t *lut, int nclass, int JP, int JPF, uint8_t *lut4,
                               int32_t *bad) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int rowb = JPF / 2;
    if (i >= (int64_t)nclass * 256 * rowb) return;
    const int64_t cr = i / rowb;                       // class * 256 + row
    const int byte = (int)(i - cr * rowb);
    const int u = byte >> 2, pair = byte & 3;          // dword u, nibbles 2*pair, 2*pair + 1
    const int U4 = JPF / 8, U8 = JP / 4;
    uint32_t out = 0;
    for (int k = 0; k < 2; ++k) {
        const int b = 2 * pair + k;
        const int jp = U4 * b + u;
        int v = 0;
        if (jp < JP) v = lut[cr * JP + 4 * (jp % U8) + jp / U8];
        const int mag = v < 0 ? -v : v;
        uint32_t code;
        switch (mag) {
        case 0: code = 0x0; break;
        case 1: code = 0x2; break;
        case 2: code = 0x4; break;
        case 3: code = 0x5; break;
        case 4: code = 0x6; break;
        case 6: code = 0x7; break;
        default: code = 0x0; atomicOr(bad, 1); break;
        }
        if (v < 0) code |= 0x8;
        out |= code << (4 * k);
    }
    lut4[i] = (uint8_t)out;
}

}  // namespace scmp

using namespace scmp;

extern "C" int scmp_build_fp4_lut(const int8_t *lut, int nclass, int JP, uint8_t *lut4,
                                  int32_t *bad, hipStream_t stream) {
    SCMP_REQUIRE(lut && lut4 && bad && nclass > 0, "scmp_build_fp4_lut: null argument");
    SCMP_REQUIRE(JP == 16 || JP == 32 || JP == 64 || JP == 128 || JP == 256,
                 "scmp_build_fp4_lut: JP=%d unsupported", JP);
    const int JPF = JP < 32 ? 32 : JP;
    const int64_t total = (int64_t)nclass * 256 * (JPF / 2);
    fp4_lut_kernel<<<cdiv(total, 256), 256, 0, stream>>>(lut, nclass, JP, JPF, lut4, bad);
    SCMP_LAUNCH_CHECK("scmp_build_fp4_lut");
    return SCMP_OK;
}
