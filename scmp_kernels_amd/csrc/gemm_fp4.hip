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

// Schedule of the non-chunked FP4 kernel (TR x TC tiles, one workgroup per CU).
struct Fp4Plan {
    int64_t tilesA, tilesB, ntiles;
    int TR, TC;               // tile rows x columns: 256 x 256, 256 x 64 (narrow), 128 x 512,
                              // 256 x 224
    int nwg;                  // persistent workgroups
    bool split;               // some tiles are shared by several workgroups
    int64_t cnt_bytes, part_bytes;
};

// Each workgroup takes an equal share of the (tile, 8-d group) work list. Tiles are shared
// only when it pays: inner dimension of at least 64 groups (512 d), and at least 32 groups
// per workgroup. Otherwise every workgroup takes whole tiles. Outputs at most 64 columns
// wide (attention's P.V per head) use 256 x 64 tiles when the stream table is a single one
// (narrow_ok), instead of computing three quarters of a 256 x 256 tile on padding. 128 x 512
// tiles are taken when they cover N x M with at least 3% less padded area than 256 x 256
// (a row count just above a multiple of 256, such as a mixed-precision level's rows).
static Fp4Plan fp4_plan(int64_t N, int64_t M, int64_t D, int64_t batch, int ncu,
                        bool narrow_ok) {
    Fp4Plan p;
    // tile counts of the two shapes (equal tile areas); wide tiles read B rows up to M
    // rounded up to 512, within the buffer only when that equals M rounded up to 256 (the
    // code buffers' row padding)
    const int64_t sq = cdiv(N, 256) * cdiv(M, 256), wide = cdiv(N, 128) * cdiv(M, 512);
    const bool wide_fits = cdiv(M, 512) * 512 == cdiv(M, 256) * 256;
    if (narrow_ok && M <= 64) {
        p.TR = 256;
        p.TC = 64;
    } else if (narrow_ok && M > 192 && M <= 224) {
        p.TR = 256;                              // 4 x 1 waves of 64 x 224
        p.TC = 224;
    } else if (wide_fits && wide * 100 <= sq * 97) {
        p.TR = 128;
        p.TC = 512;
    } else {
        p.TR = 256;
        p.TC = 256;
    }
    p.tilesA = cdiv(N, p.TR);
    p.tilesB = cdiv(M, p.TC);
    p.ntiles = p.tilesA * p.tilesB * batch;
    const int64_t G = cdiv(D, 8);
    const int64_t W = p.ntiles * G;
    int64_t nwg = p.ntiles;                      // whole tiles, one per workgroup
    // a whole number of 256-wide tiles per compute unit (attention's 768 QK^T heads on 256):
    // persistent workgroups take them in turn and load their tables once (QK^T 5% faster;
    // the narrow P.V tiles measured 9% slower that way, so they keep one per workgroup)
    if (p.TC != 64 && p.ntiles > ncu && p.ntiles % ncu == 0) nwg = ncu;
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
    p.part_bytes = (int64_t)p.nwg * 2 * (p.TR * p.TC) * 4;
    return p;
}

__global__ void zero_ints_kernel(int *p, int64_t n) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Narrow tiles are instantiated for a single stream table in LDS (no per-d classes).
static bool fp4_narrow_ok(const scmp_gemm_args &a) {
    return a.d_class == nullptr && a.group_class == nullptr;
}

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
    if (chunked) {
        P.nwg = device_cu_count();               // sizes the rounds of whole tiles
        return fp4_launch_jpf(P, a.batch, a.JP < 32 ? 32 : a.JP, true, stream);
    }
    const int JPF = a.JP;
    Fp4Plan plan = fp4_plan(a.N, a.M, a.D, a.batch, device_cu_count(), fp4_narrow_ok(a));
    P.tile_cols = plan.TC;
    P.tilesA = (int)plan.tilesA;
    P.tilesB = (int)plan.tilesB;
    P.ntiles = plan.ntiles;
    P.part = nullptr;
    P.cnt = nullptr;
    P.deferred = 0;
    P.nwg = (int)plan.ntiles;                 // whole tiles unless the workspace allows splits
    if (plan.split && a.workspace && a.workspace_bytes >= plan.cnt_bytes + plan.part_bytes) {
        P.nwg = plan.nwg;
        P.cnt = (int *)a.workspace;
        P.part = (float *)((uint8_t *)a.workspace + plan.cnt_bytes);
        // Fewer tiles than workgroups: most tiles have three or more contributors, which all
        // finish at the end of the launch, so the last to arrive would add two or more slots
        // and drain the tile while the rest of the chip idles. Those tiles are finished by a
        // second launch over every compute unit instead (no counters).
        P.deferred = plan.ntiles < plan.nwg ? 1 : 0;
        if (!P.deferred) {
            zero_ints_kernel<<<cdiv(plan.ntiles, 256), 256, 0, stream>>>(P.cnt, plan.ntiles);
            SCMP_LAUNCH_CHECK("scmp_sc_gemm(fp4 counters)");
        }
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
        const int jp = 8 * u + b;
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

// Code columns in class runs, any row stride: thread (r, 16-byte chunk p0) writes
// out[r][p0 .. p0 + 15] from bytes of row r read through the cache.
__global__ void permute_columns_kernel(const uint8_t *in, int64_t rows, int64_t ld_in,
                                       const int32_t *src, int64_t ncols, uint8_t *out,
                                       int64_t ld_out) {
    const int64_t chunks = ld_out / 16;
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= rows * chunks) return;
    const int64_t r = i / chunks, p0 = 16 * (i - r * chunks);
    const uint8_t *row = in + r * ld_in;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int64_t p = p0 + k;
        const int32_t c = p < ncols ? src[p] : -1;
        if (c >= 0) w[k >> 2] |= (uint32_t)row[c] << (8 * (k & 3));
    }
    *(uint4 *)(out + r * ld_out + p0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Row strides that are multiples of 16 (code buffers): RW rows per workgroup are read
// whole into LDS with 16-byte loads, then each thread gathers 16-byte output chunks from
// LDS, reading its 16 source indices once for the RW rows.
template <int RW>
__global__ void __launch_bounds__(256)
permute_columns_lds_kernel(const uint8_t *in, int64_t rows, int64_t ld_in, const int32_t *src,
                           int64_t ncols, uint8_t *out, int64_t ld_out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t srow[];
    const int64_t r0 = (int64_t)blockIdx.x * RW;
    const int nr = rows - r0 < RW ? (int)(rows - r0) : RW;
    const int cin = (int)(ld_in / 16);
    for (int e = threadIdx.x; e < nr * cin; e += 256) {
        const int k = e / cin, c = e - k * cin;
        *(uint4 *)(srow + (int64_t)k * ld_in + 16 * c) =
            *(const uint4 *)(in + (r0 + k) * ld_in + 16 * c);
    }
    __syncthreads();
    const int cout = (int)(ld_out / 16);
    for (int c = threadIdx.x; c < cout; c += 256) {
        const int64_t p0 = 16 * (int64_t)c;
        int32_t s[16];
        if (p0 + 16 <= ncols) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int4 v = *(const int4 *)(src + p0 + 4 * q);
                s[4 * q] = v.x; s[4 * q + 1] = v.y; s[4 * q + 2] = v.z; s[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) s[k] = p0 + k < ncols ? src[p0 + k] : -1;
        }
        for (int k = 0; k < nr; ++k) {
            const uint8_t *row = srow + (int64_t)k * ld_in;
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (s[j] >= 0) w[j >> 2] |= (uint32_t)row[s[j]] << (8 * (j & 3));
            *(uint4 *)(out + (r0 + k) * ld_out + p0) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

extern "C" int scmp_permute_code_columns(const uint8_t *in, int64_t rows, int64_t ld_in,
                                         const int32_t *src, int64_t ncols, uint8_t *out,
                                         int64_t ld_out, hipStream_t stream) {
    SCMP_REQUIRE(in && src && out, "scmp_permute_code_columns: null pointer");
    SCMP_REQUIRE(rows > 0 && ncols > 0 && ld_in > 0 && ld_out % 16 == 0 && ld_out >= ncols,
                 "scmp_permute_code_columns: rows=%lld ncols=%lld ld_in=%lld ld_out=%lld "
                 "(ld_out a multiple of 16, >= ncols)", (long long)rows, (long long)ncols,
                 (long long)ld_in, (long long)ld_out);
    const bool aligned = ld_in % 16 == 0 && ((uintptr_t)in & 15) == 0 &&
                         ((uintptr_t)out & 15) == 0 && ((uintptr_t)src & 15) == 0;
    if (aligned && ld_in <= 16384) {
        permute_columns_lds_kernel<4><<<cdiv(rows, 4), 256, 4 * ld_in, stream>>>(
            in, rows, ld_in, src, ncols, out, ld_out);
    } else if (aligned && ld_in <= 65536) {
        permute_columns_lds_kernel<1><<<rows, 256, ld_in, stream>>>(in, rows, ld_in, src, ncols,
                                                                   out, ld_out);
    } else {
        const int64_t n = rows * (ld_out / 16);
        permute_columns_kernel<<<cdiv(n, 256), 256, 0, stream>>>(in, rows, ld_in, src, ncols,
                                                                 out, ld_out);
    }
    SCMP_LAUNCH_CHECK("scmp_permute_code_columns");
    return SCMP_OK;
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
