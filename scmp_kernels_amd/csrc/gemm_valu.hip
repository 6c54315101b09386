// SC GEMM on the vector ALUs: bit-packed stream words, AND + popcount (v_bcnt_u32_b32).
//
// Same integer I[n,m] as the MFMA kernel (gemm_mfma.hip) and the same operand codes:
// per (n, m, d) the A-side thermometer of j_a intervals is ANDed with the two bit planes
// of the B-side interval counts (counts are 0..3, so two planes suffice) and popcounted:
//   count = popc(T & P0) + 2 * popc(T & P1),  I += s_a * s_b * count.
// This is the textbook bitstream formulation the reference describes ("XNOR/AND +
// popcount"); it exists to be measured against the MFMA kernel, which replaces it as the
// default (see the rocprof comparison kept under profiles/).
//
// Each thread owns a 4 x 4 output micro-tile; a 256-thread workgroup covers 64 x 64.
// Codes for 16 values of d at a time are staged through LDS; the bit-plane table of a
// shared class lives in LDS for the whole kernel.
#include "gemm_common.h"

namespace scmp {

template <int W>  // words per plane (JP / 32, at least 1)
__global__ void __launch_bounds__(256)
sc_gemm_valu_kernel(const uint8_t *ca, int64_t lda, int64_t bsa, const uint8_t *cb,
                    int64_t ldb, int64_t bsb, int N, int M, int D, int JP, int bipolar,
                    const uint32_t *bitlut, const int32_t *d_class, scmp_epilogue E,
                    float *y, int32_t *iout, int64_t ldy, int64_t bsy, int tilesA,
                    const int64_t *row_map) {
    __shared__ uint32_t sbits[256 * 2 * W];
    __shared__ uint8_t sa_codes[64][17];
    __shared__ uint8_t sb_codes[64][17];
    const int tid = threadIdx.x;
    if (!d_class)
        for (int e = tid; e < 256 * 2 * W; e += 256) sbits[e] = bitlut[e];
    const int ta = blockIdx.x % tilesA, tb = blockIdx.x / tilesA, batch = blockIdx.z;
    const int a0 = ta * 64, b0 = tb * 64;
    const int tx = tid & 15, ty = tid >> 4;     // rows a0 + 4ty + i, cols b0 + 4tx + c
    int32_t acc[4][4] = {};
    const uint8_t *A = ca + batch * bsa;
    const uint8_t *B = cb + batch * bsb;
    for (int d0 = 0; d0 < D; d0 += 16) {
        __syncthreads();
        for (int e = tid; e < 64 * 16; e += 256) {
            int r = e >> 4, k = e & 15;
            sa_codes[r][k] = A[(int64_t)(a0 + r) * lda + d0 + k];
            sb_codes[r][k] = B[(int64_t)(b0 + r) * ldb + d0 + k];
        }
        __syncthreads();
        const int dn = D - d0 < 16 ? D - d0 : 16;
        for (int k = 0; k < dn; ++k) {
            const uint32_t *tab = d_class ? bitlut + (int64_t)d_class[d0 + k] * 256 * 2 * W : sbits;
            int ja[4], sgn_a[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int code = sa_codes[4 * ty + i][k];
                ja[i] = bipolar ? (code & 0x7f) : code;
                sgn_a[i] = (bipolar && (code & 0x80)) ? -1 : 1;
            }
            uint32_t p0[4][W], p1[4][W];
            int sgn_b[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                int code = sb_codes[4 * tx + c][k];
                sgn_b[c] = (bipolar && (code & 0x80)) ? -1 : 1;
                const uint32_t *row = tab + code * 2 * W;
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    p0[c][w] = row[w];
                    p1[c][w] = row[W + w];
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    int bits = ja[i] - 32 * w;
                    uint32_t t = bits >= 32 ? 0xffffffffu : (bits <= 0 ? 0u : ((1u << bits) - 1u));
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        int cnt = __builtin_popcount(t & p0[c][w]) +
                                  2 * __builtin_popcount(t & p1[c][w]);
                        acc[i][c] += sgn_a[i] * sgn_b[c] * cnt;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = a0 + 4 * ty + i;
        if (n >= N) continue;
        const int64_t row = out_row(row_map, n);     // one row-map load per row
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int m = b0 + 4 * tx + c;
            if (m >= M) continue;
            const int64_t o = batch * bsy + row * ldy + m;
            const int I = acc[i][c];
            if (E.kind == SCMP_EPI_INT) iout[o] = I;
            else y[o] = epilogue_value(E, (float)I, n, m, batch);
        }
    }
}

int gemm_valu_launch(const scmp_gemm_args &a, hipStream_t stream) {
    SCMP_REQUIRE(a.bitlut != nullptr, "scmp_sc_gemm(valu): bitlut required");
    SCMP_REQUIRE(a.chunk <= 0 || a.chunk >= a.D, "scmp_sc_gemm(valu): no chunked mode");
    const int tilesA = (int)cdiv(a.N, 64);
    const int64_t tilesB = cdiv(a.M, 64);
    dim3 grid((unsigned)(tilesA * tilesB), 1, (unsigned)a.batch);
    const int W = a.JP / 32 > 0 ? a.JP / 32 : 1;
#define SCMP_VALU_CASE(WW)                                                                   \
    case WW:                                                                                 \
        sc_gemm_valu_kernel<WW><<<grid, 256, 0, stream>>>(                                   \
            a.ca, a.lda, a.bsa, a.cb, a.ldb, a.bsb, (int)a.N, (int)a.M, (int)a.D, a.JP,      \
            a.bipolar, a.bitlut, a.d_class, a.epi, a.y, a.iout, a.ldy, a.bsy, tilesA,        \
            a.row_map);                                                                      \
        break;
    switch (W) {
        SCMP_VALU_CASE(1)
        SCMP_VALU_CASE(2)
        SCMP_VALU_CASE(4)
        SCMP_VALU_CASE(8)
    default: set_error("scmp_sc_gemm(valu): JP=%d unsupported", a.JP); return SCMP_E_ARG;
    }
#undef SCMP_VALU_CASE
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(valu)");
    return SCMP_OK;
}

}  // namespace scmp
