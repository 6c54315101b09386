// FP4 (e2m1) SC GEMM: dispatch over the table width, and the FP4 form of a stream table.
// The kernel itself is in gemm_fp4_kernel.h.
#include "gemm_common.h"

namespace scmp {

// Compute units of the current device (cached per device).
static int device_cu_count() {
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

// Schedule of the non-chunked FP4 kernel (256 x TC tiles, one workgroup per CU).
struct Fp4Plan {
    int64_t tilesA, tilesB, ntiles;
    int TC;                   // tile columns: 256, or 64 when M <= 64 (narrow tiles)
    int nwg;                  // persistent workgroups
    bool split;               // some tiles are shared by several workgroups
    int64_t cnt_bytes, part_bytes;
};

// Each workgroup takes an equal share of the (tile, 8-d group) work list. Tiles are shared
// only when it pays: inner dimension of at least 64 groups (512 d), and at least 32 groups
// per workgroup. Otherwise every workgroup takes whole tiles. Outputs at most 64 columns
// wide (attention's P.V per head) use 256 x 64 tiles when the stream table is a single one
// (narrow_ok), instead of computing three quarters of a 256 x 256 tile on padding.
static Fp4Plan fp4_plan(int64_t N, int64_t M, int64_t D, int64_t batch, int ncu,
                        bool narrow_ok) {
    Fp4Plan p;
    p.TC = narrow_ok && M <= 64 ? 64 : 256;
    p.tilesA = cdiv(N, 256);
    p.tilesB = cdiv(M, p.TC);
    p.ntiles = p.tilesA * p.tilesB * batch;
    const int64_t G = cdiv(D, 8);
    const int64_t W = p.ntiles * G;
    int64_t nwg = p.ntiles;                      // whole tiles, one per workgroup
    if (G >= 64) {
        if (p.ntiles >= ncu) {
            nwg = ncu;
        } else {
            nwg = W / 32;
            if (nwg > ncu) nwg = ncu;
            if (nwg < p.ntiles) nwg = p.ntiles;
        }
    }
    p.nwg = (int)nwg;
    p.split = (W % p.nwg) != 0 || (W / p.nwg) % G != 0;
    p.cnt_bytes = (p.ntiles * 4 + 255) / 256 * 256;
    p.part_bytes = (int64_t)p.nwg * 2 * (256 * p.TC) * 4;
    return p;
}

__global__ void zero_ints_kernel(int *p, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Narrow tiles are instantiated for a single stream table in LDS (no per-d classes).
static bool fp4_narrow_ok(const scmp_gemm_args &a) { return a.d_class == nullptr; }

static int fp4_launch_jpf(const GemmP &P, int64_t batch, int JPF, bool chunked,
                          hipStream_t stream) {
    switch (JPF) {
    case 16: return gemm_fp4_launch_jpf<16>(P, batch, chunked, stream);
    case 32: return gemm_fp4_launch_jpf<32>(P, batch, chunked, stream);
    case 64: return gemm_fp4_launch_jpf<64>(P, batch, chunked, stream);
    case 128: return gemm_fp4_launch_jpf<128>(P, batch, chunked, stream);
    case 256: return gemm_fp4_launch_jpf<256>(P, batch, chunked, stream);
    default: set_error("scmp_sc_gemm(fp4): JPF=%d unsupported", JPF); return SCMP_E_ARG;
    }
}

int gemm_fp4_run(GemmP &P, const scmp_gemm_args &a, bool chunked, hipStream_t stream) {
    // 16-interval tables: four inner dimensions per MFMA k-step (JPF = 16), except in the
    // chunk_d kernel, whose chunk boundaries need only be even (JPF = 32)
    if (chunked) return fp4_launch_jpf(P, a.batch, a.JP < 32 ? 32 : a.JP, true, stream);
    const int JPF = a.JP;
    Fp4Plan plan = fp4_plan(a.N, a.M, a.D, a.batch, device_cu_count(), fp4_narrow_ok(a));
    P.tile_cols = plan.TC;
    P.tilesA = (int)plan.tilesA;
    P.tilesB = (int)plan.tilesB;
    P.ntiles = plan.ntiles;
    P.part = nullptr;
    P.cnt = nullptr;
    P.nwg = (int)plan.ntiles;                 // whole tiles unless the workspace allows splits
    if (plan.split && a.workspace && a.workspace_bytes >= plan.cnt_bytes + plan.part_bytes) {
        P.nwg = plan.nwg;
        P.cnt = (int *)a.workspace;
        P.part = (float *)((uint8_t *)a.workspace + plan.cnt_bytes);
        zero_ints_kernel<<<cdiv(plan.ntiles, 256), 256, 0, stream>>>(P.cnt, plan.ntiles);
        SCMP_LAUNCH_CHECK("scmp_sc_gemm(fp4 counters)");
    } else if (!plan.split) {
        P.nwg = plan.nwg;                     // an even share of whole tiles each
    }
    return fp4_launch_jpf(P, a.batch, JPF, false, stream);
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
    const int U4 = JP < JPF ? JP / 8 : JPF / 8, U8 = JP / 4;   // dwords holding intervals
    uint32_t out = 0;
    for (int k = 0; k < 2; ++k) {
        const int b = 2 * pair + k;
        const int jp = U4 * b + u;
        int v = 0;
        if (u < U4 && jp < JP) v = lut[cr * JP + 4 * (jp % U8) + jp / U8];
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

extern "C" int64_t scmp_sc_gemm_workspace_bytes(const scmp_gemm_args *a) {
    if (!a || a->impl != SCMP_GEMM_MFMA_FP4 || a->N <= 0 || a->M <= 0 || a->D <= 0 ||
        a->batch <= 0 || (a->chunk > 0 && a->chunk < a->D))
        return 0;
    const Fp4Plan p = fp4_plan(a->N, a->M, a->D, a->batch, device_cu_count(), fp4_narrow_ok(*a));
    return p.split ? p.cnt_bytes + p.part_bytes : 0;
}

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
