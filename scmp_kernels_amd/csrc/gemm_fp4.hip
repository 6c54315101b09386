// FP4 (e2m1) SC GEMM: dispatch over the table width, and the FP4 form of a stream table.
// The kernel itself is in gemm_fp4_kernel.h.
#include "gemm_common.h"

namespace scmp {

int gemm_fp4_launch(const GemmP &P, int64_t batch, int JPF, bool chunked, hipStream_t stream) {
    switch (JPF) {
    case 32: return gemm_fp4_launch_jpf<32>(P, batch, chunked, stream);
    case 64: return gemm_fp4_launch_jpf<64>(P, batch, chunked, stream);
    case 128: return gemm_fp4_launch_jpf<128>(P, batch, chunked, stream);
    case 256: return gemm_fp4_launch_jpf<256>(P, batch, chunked, stream);
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
