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
#include "gemm_common.h"

namespace scmp {

__device__ __forceinline__ v16i mfma_i8(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v16c, a),
                                                 __builtin_bit_cast(v16c, b), c, 0, 0, 0);
}

// (FULL, PART) dword pair of a thermometer code, computed in registers: j = code & 0x7f
// (bipolar, sign in bit 7) or code (unipolar); qq = j / (JP/4); FULL has the sign byte in
// bytes b < qq, PART also in byte qq (equal to FULL when qq == 4, i.e. j == JP).
template <int JP>
__device__ __forceinline__ void thermo_pair(int code, bool bipolar, uint32_t &full,
                                            uint32_t &part, int &rr, int h) {
    constexpr int U = JP / 4;
    const int j = bipolar ? (code & 0x7f) : code;
    const int qq = j / U;
    const uint32_t neg = bipolar ? (uint32_t)((int)((uint32_t)code << 24) >> 31) : 0u;
    const uint32_t spat = neg | 0x01010101u;
    const int w = 8 * qq;
    const uint32_t m = qq >= 4 ? 0xffffffffu : ((1u << (w & 31)) - 1u);
    full = m & spat;
    part = qq >= 4 ? full : (full | (spat & (0xffu << (w & 31))));
    rr = JP == 16 ? (j & 3) : ((j & (U - 1)) - 4 * h);
}

template <int JP, int BA, int BB, int WA, int WB, bool PERCLASS, bool CHUNKED, bool PIPE>
__global__ void __launch_bounds__(64 * WA * WB)
sc_gemm_mfma_kernel(GemmP P) {
    constexpr int NT = 64 * WA * WB;
    constexpr int U = JP / 4;                  // dwords per row
    constexpr int KSTEPS = JP >= 32 ? JP / 32 : 1;
    // LUT rows in LDS are an odd number of 16-byte chunks apart: with a stride that is a
    // multiple of the 128-byte bank width every row would start in bank 0, and the 16-byte
    // B-operand reads of one k-step (same offset, data-dependent rows) would all hit the
    // same four banks; an odd chunk stride spreads row starts over all eight bank groups.
    constexpr int LSTRIDE = 16 * ((JP / 16) | 1);
    __shared__ __attribute__((aligned(16))) int8_t slut[PERCLASS ? 16 : 256 * LSTRIDE];

    const int tid = threadIdx.x;
    if (!PERCLASS) {
        const v4i *src = (const v4i *)P.lut;
        for (int e = tid; e < 256 * JP / 16; e += NT) {
            const int row = e / (JP / 16), col = e - row * (JP / 16);
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
                    float raw = __fmul_rn((float)acc[i][c][r], cc);
                    float term = __fmul_rn(raw, __fmul_rn(san, sbm));
                    yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r] =
                        __fadd_rn(yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r], term);
                    acc[i][c][r] = 0;
                }
        }
        ++kchunk;
    };

    if constexpr (JP >= 32 && !PIPE) {
        // d loop without cross-d prefetch: the LDS reads of each k-step are issued just
        // before its MFMAs (the compiler interleaves the A-operand VALU work with them).
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
#pragma unroll 1
            for (int dd = 0; dd < 8; ++dd) {
                const int sh = 8 * dd;
                uint32_t full[BA], part[BA];
                int rr[BA];
#pragma unroll
                for (int i = 0; i < BA; ++i)
                    thermo_pair<JP>((int)((ca8[i] >> sh) & 0xff), P.bipolar, full[i], part[i],
                                    rr[i], h);
                const int8_t *lp[BB];
                const int8_t *base;
                if (PERCLASS) {
                    const int dcur = dbase + dd;
                    const int cls = (P.d_class && dcur < D) ? P.d_class[dcur] : 0;
                    base = P.lut + (int64_t)cls * 256 * JP;
                } else {
                    base = slut;
                }
#pragma unroll
                for (int c = 0; c < BB; ++c)
                    lp[c] = base + (int)((cb8[c] >> sh) & 0xff) * (PERCLASS ? JP : LSTRIDE) +
                            16 * h;
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
                if (CHUNKED) flush_chunk(dbase + dd);
            }
        }
    } else if constexpr (JP >= 32) {
        // Software-pipelined d loop: while the MFMAs of dimension d run, the LDS reads of
        // d + 1 (thermometer (FULL, PART) pairs and B-operand LUT rows) are in flight.
        constexpr bool PREF_B = KSTEPS * BB * 4 <= 32;   // register budget for prefetched rows
        struct DState {
            uint32_t full[BA], part[BA];
            int rr[BA];
            const int8_t *lp[BB];
            v4i bf[PREF_B ? KSTEPS : 1][BB];
        };
        DState st[2];
        auto load_d = [&](DState &S, const uint32_t (&cw_a)[BA], const uint32_t (&cw_b)[BB],
                          int byte, int d) {
#pragma unroll
            for (int i = 0; i < BA; ++i) {
                const int code = (int)((cw_a[i] >> (8 * byte)) & 0xff);
                thermo_pair<JP>(code, P.bipolar, S.full[i], S.part[i], S.rr[i], h);
            }
            const int8_t *base;
            if (PERCLASS) {
                const int cls = (P.d_class && d < D) ? P.d_class[d] : 0;
                base = P.lut + (int64_t)cls * 256 * JP;
            } else {
                base = slut;
            }
#pragma unroll
            for (int c = 0; c < BB; ++c) {
                const int code = (int)((cw_b[c] >> (8 * byte)) & 0xff);
                S.lp[c] = base + code * (PERCLASS ? JP : LSTRIDE) + 16 * h;
                if (PREF_B) {
#pragma unroll
                    for (int t = 0; t < (PREF_B ? KSTEPS : 1); ++t)
                        S.bf[t][c] = *(const v4i *)(S.lp[c] + 32 * t);
                }
            }
        };
        auto compute_d = [&](DState &S) {
#pragma unroll
            for (int t = 0; t < KSTEPS; ++t) {
                v4i bf[BB];
#pragma unroll
                for (int c = 0; c < BB; ++c)
                    bf[c] = PREF_B ? S.bf[PREF_B ? t : 0][c] : *(const v4i *)(S.lp[c] + 32 * t);
#pragma unroll
                for (int i = 0; i < BA; ++i) {
                    v4i af;
                    af.x = (8 * t + 0 < S.rr[i]) ? S.part[i] : S.full[i];
                    af.y = (8 * t + 1 < S.rr[i]) ? S.part[i] : S.full[i];
                    af.z = (8 * t + 2 < S.rr[i]) ? S.part[i] : S.full[i];
                    af.w = (8 * t + 3 < S.rr[i]) ? S.part[i] : S.full[i];
#pragma unroll
                    for (int c = 0; c < BB; ++c) acc[i][c] = mfma_i8(af, bf[c], acc[i][c]);
                }
            }
        };
        uint32_t wa_lo[BA], wa_hi[BA], wb_lo[BB], wb_hi[BB];
#pragma unroll
        for (int i = 0; i < BA; ++i) { wa_lo[i] = na[i].x; wa_hi[i] = na[i].y; }
#pragma unroll
        for (int c = 0; c < BB; ++c) { wb_lo[c] = nb[c].x; wb_hi[c] = nb[c].y; }
        load_d(st[0], wa_lo, wb_lo, 0, 0);
        for (int g = 0; g < ngroups; ++g) {
            const bool more = g + 1 < ngroups;
            if (more) {
#pragma unroll
                for (int i = 0; i < BA; ++i) na[i] = *(const uint2 *)(pa[i] + 8 * (g + 1));
#pragma unroll
                for (int c = 0; c < BB; ++c) nb[c] = *(const uint2 *)(pb[c] + 8 * (g + 1));
            }
            const int dbase = 8 * g;
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) {
                DState &cur = st[dd & 1];
                DState &nxt = st[(dd + 1) & 1];
                if (dd < 3) load_d(nxt, wa_lo, wb_lo, dd + 1, dbase + dd + 1);
                else if (dd < 7) load_d(nxt, wa_hi, wb_hi, dd - 3, dbase + dd + 1);
                else if (more) {
#pragma unroll
                    for (int i = 0; i < BA; ++i) { wa_lo[i] = na[i].x; wa_hi[i] = na[i].y; }
#pragma unroll
                    for (int c = 0; c < BB; ++c) { wb_lo[c] = nb[c].x; wb_hi[c] = nb[c].y; }
                    load_d(nxt, wa_lo, wb_lo, 0, dbase + 8);
                }
                compute_d(cur);
                if (CHUNKED) flush_chunk(dbase + dd);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // JP == 16: two inner dimensions per k-step (lane half h takes d = 2p + h)
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
#pragma unroll 1
            for (int dd = 0; dd < 8; dd += 2) {
                const int sh = 8 * (dd + h);
                uint32_t full[BA], part[BA];
                int rr[BA];
#pragma unroll
                for (int i = 0; i < BA; ++i) {
                    const int code = (int)((ca8[i] >> sh) & 0xff);
                    thermo_pair<JP>(code, P.bipolar, full[i], part[i], rr[i], h);
                }
                v4i bf[BB];
#pragma unroll
                for (int c = 0; c < BB; ++c) {
                    const int code = (int)((cb8[c] >> sh) & 0xff);
                    const int8_t *base;
                    if (PERCLASS) {
                        const int dcur = dbase + dd + h;
                        const int cls = (P.d_class && dcur < D) ? P.d_class[dcur] : 0;
                        base = P.lut + (int64_t)cls * 256 * JP;
                    } else {
                        base = slut;
                    }
                    bf[c] = *(const v4i *)(base + code * (PERCLASS ? JP : LSTRIDE));
                }
#pragma unroll
                for (int i = 0; i < BA; ++i) {
                    v4i af;
                    af.x = (0 < rr[i]) ? part[i] : full[i];
                    af.y = (1 < rr[i]) ? part[i] : full[i];
                    af.z = (2 < rr[i]) ? part[i] : full[i];
                    af.w = (3 < rr[i]) ? part[i] : full[i];
#pragma unroll
                    for (int c = 0; c < BB; ++c) acc[i][c] = mfma_i8(af, bf[c], acc[i][c]);
                }
                if (CHUNKED && dbase + dd < D) flush_chunk(dbase + dd + 1 < D ? dbase + dd + 1 : D - 1);
            }
        }
    }

    // ---------------- store ----------------
    // Non-chunked kernels store the exact int32 I; the fp32 epilogue runs as a separate
    // elementwise pass (epilogue_kernel, in place over the same buffer). Fusing it here
    // makes the register allocator move all accumulators out of the AGPRs and spill.
    // One loop per row mapping, so that the common one (no row map) issues no loads
    // between its stores (a load's wait would also wait for every store before it).
    auto store_all = [&](auto row_of) __attribute__((always_inline)) {
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
                    const int64_t o = batch * P.bsy + row_of(n) * P.ldy + m;
                    if (CHUNKED) {
                        P.y[o] = yac[CHUNKED ? i : 0][CHUNKED ? c : 0][r];
                        continue;
                    }
                    P.iout[o] = acc[i][c][r];
                }
            }
        }
    };
    if (P.row_map == nullptr)
        store_all([](int n) { return (int64_t)n; });
    else
        store_all([&](int n) { return P.row_map[n]; });
}

// fp32 epilogues of the reference paths, applied to the int32 accumulator in place
// (int8 MFMA and VALU kernels; the FP4 kernel applies them itself).
__global__ void epilogue_kernel(const int32_t *iin, float *y, int N, int M, int64_t ldy,
                                int64_t bsy, scmp_epilogue E, const int64_t *row_map) {
    const int batch = blockIdx.z;
    for (int n = blockIdx.y; n < N; n += gridDim.y)
    for (int m = blockIdx.x * blockDim.x + threadIdx.x; m < M; m += gridDim.x * blockDim.x) {
        const int64_t o = batch * bsy + out_row(row_map, n) * ldy + m;
        y[o] = epilogue_value(E, (float)iin[o], n, m, batch);
    }
}

int run_epilogue(const int32_t *iin, float *y, int64_t N, int64_t M, int64_t batch,
                 int64_t ldy, int64_t bsy, const scmp_epilogue &E, const int64_t *row_map,
                 hipStream_t stream) {
    int64_t bx = cdiv(M, 256);
    if (bx > 64) bx = 64;
    dim3 grid((unsigned)bx, (unsigned)(N < 32768 ? N : 32768), (unsigned)batch);
    epilogue_kernel<<<grid, 256, 0, stream>>>(iin, y, (int)N, (int)M, ldy, bsy, E, row_map);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(epilogue)");
    return SCMP_OK;
}

template <int JP, int BA, int BB, int WA, int WB, bool PERCLASS, bool CHUNKED, bool PIPE>
static int launch_t(const GemmP &P0, int64_t batch, hipStream_t stream) {
    GemmP P = P0;
    const int tileA = WA * BA * 32, tileB = WB * BB * 32;
    P.tilesA = (int)cdiv(P.N, tileA);
    const int64_t tilesB = cdiv(P.M, tileB);
    dim3 grid((unsigned)(P.tilesA * tilesB), 1, (unsigned)batch);
    sc_gemm_mfma_kernel<JP, BA, BB, WA, WB, PERCLASS, CHUNKED, PIPE>
        <<<grid, 64 * WA * WB, 0, stream>>>(P);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma)");
    return SCMP_OK;
}

// Tile presets: rows of A (thermometer side) x rows of B (LUT side) per workgroup.
//  0: 256 x 256, each wave 256 x 64 (8 x 2 blocks of 32x32, 256 accumulator registers)
//  1: 256 x 128, each wave 128 x 64 (4 x 2 blocks, two waves per SIMD fit)
//  2: 256 x 256, each wave 128 x 128 (4 x 4 blocks)
//  3, 4: presets 0 and 2 with the software-pipelined d loop
//  chunked epilogue: 128 x 128, each wave 64 x 64 (2 x 2 blocks, fp32 sums in registers)
template <int JP, bool PERCLASS>
static int launch_jp(const GemmP &P, int64_t batch, int tile, bool chunked, hipStream_t s) {
    if (chunked) return launch_t<JP, 2, 2, 2, 2, PERCLASS, true, false>(P, batch, s);
    switch (tile) {
    case 1: return launch_t<JP, 4, 2, 2, 2, PERCLASS, false, false>(P, batch, s);
    case 2: return launch_t<JP, 4, 4, 2, 2, PERCLASS, false, false>(P, batch, s);
    case 3: return launch_t<JP, 8, 2, 1, 4, PERCLASS, false, true>(P, batch, s);
    case 4: return launch_t<JP, 4, 4, 2, 2, PERCLASS, false, true>(P, batch, s);
    default: return launch_t<JP, 8, 2, 1, 4, PERCLASS, false, false>(P, batch, s);
    }
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
    // |I| <= 256 * D: int32 accumulators stay exact below D = 2^23
    SCMP_REQUIRE(a.N < (1LL << 30) && a.M < (1LL << 30) && a.D < (1LL << 23) &&
                     a.batch < 65536,
                 "scmp_sc_gemm: dimensions too large");
    // the FP4 kernel accumulates in fp32, exact for integers up to 2^24 = 256 * 65536
    SCMP_REQUIRE(a.impl != SCMP_GEMM_MFMA_FP4 || a.D <= 65536,
                 "scmp_sc_gemm: D=%lld exceeds the exact fp32 range of the FP4 kernel",
                 (long long)a.D);
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
    SCMP_REQUIRE(!chunked || a.impl != SCMP_GEMM_VALU,
                 "scmp_sc_gemm: chunked accumulation is implemented by the MFMA kernels");
    SCMP_REQUIRE(a.group_class == nullptr ||
                     (a.impl == SCMP_GEMM_MFMA_FP4 && !chunked && a.d_class == nullptr &&
                      a.D % 8 == 0 && a.nclass > 0),
                 "scmp_sc_gemm: group_class needs the FP4 kernel, no chunked accumulation, "
                 "no d_class, D a multiple of 8 and nclass > 0");
    if (a.impl == SCMP_GEMM_VALU) return gemm_valu_launch(a, stream);
    SCMP_REQUIRE(a.impl == SCMP_GEMM_MFMA || a.impl == SCMP_GEMM_MFMA_FP4,
                 "scmp_sc_gemm: unknown impl %d", a.impl);
    GemmP P;
    P.ca = a.ca; P.lda = a.lda; P.bsa = a.bsa;
    P.cb = a.cb; P.ldb = a.ldb; P.bsb = a.bsb;
    P.N = (int)a.N; P.M = (int)a.M; P.D = (int)a.D;
    P.chunk = chunked ? (int)a.chunk : 0;
    P.lut = a.lut; P.d_class = a.d_class; P.bipolar = a.bipolar; P.JP = a.JP;
    P.epi = a.epi; P.y = a.y; P.ldy = a.ldy; P.bsy = a.bsy;
    P.row_map = a.row_map;
    P.group_class = a.group_class;
    P.row0 = 0;
    P.deferred = 0;
    P.tilesA = 0;
    P.tile_cols = 256;
    P.nclass = a.nclass;
    if (a.impl == SCMP_GEMM_MFMA_FP4) {
        // the FP4 kernel applies the epilogue itself (int32 I for SCMP_EPI_INT)
        P.iout = a.iout;
        return gemm_fp4_run(P, a, chunked, stream);
    }
    // int8 MFMA, non-chunked: int32 I goes to iout, or into the fp32 output buffer itself
    // (the epilogue pass then converts it in place)
    P.iout = a.epi.kind == SCMP_EPI_INT ? a.iout : (int32_t *)a.y;
    const bool perclass = a.d_class != nullptr;
    const int rc = perclass ? launch_pc<true>(P, a.batch, a.JP, a.tile, chunked, stream)
                            : launch_pc<false>(P, a.batch, a.JP, a.tile, chunked, stream);
    if (rc != SCMP_OK || chunked || a.epi.kind == SCMP_EPI_INT) return rc;
    return run_epilogue(P.iout, a.y, a.N, a.M, a.batch, a.ldy, a.bsy, a.epi, a.row_map,
                        stream);
}
