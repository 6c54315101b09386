// SC GEMM kernels on the gfx950 matrix cores with FP4 (e2m1) operands:
// v_mfma_scale_f32_32x32x64_f8f6f4 (cbsz = blgp = 4, unit scales), twice the int8 rate.
//
// Same product as the int8 kernel (gemm_mfma.hip): I[n,m] = sum_d sum_{j' < JPF}
// thermo(code_a)[j'] * lut[class(d)][code_b][j']. Every operand value is a small integer
// that e2m1 represents exactly: the A side is 0 or +-1.0 (nibbles 0x0, 0x2, 0xA), the B
// side an interval count 0..4 or 6 (0x0 0x2 0x4 0x5 0x6 0x7, sign bit 0x8). Products and
// every partial sum are integers of magnitude <= 256 * D <= 2^24 (the host limits D to
// 65536), so the fp32 accumulation is exact and (int)acc == I; partial sums of disjoint
// inner-dimension ranges add exactly in any order.
//
// One MFMA covers K = 64 intervals (lane half h: 32 nibbles = 4 dwords). Layout of one
// table row of JP intervals (JP >= 32): dword u (JP/8 of them), nibble b holds interval
// j' = 8u + b (any order of the intervals gives the same sums as long as both operands use
// it; the contiguous one measured ~1% faster than an interleaved one, through the MFMA
// clock, which depends on operand bit activity); k-step t, lane half h holds dwords
// u = 8t + 4h + w. JPF = 32 puts two inner dimensions in one k-step (half h takes
// d = 2p + h). A 16-interval table is stored in 32-interval rows: dwords 0-1 hold its
// intervals, dwords 2-3 are zero; JPF = 16 reads
// just those 8 bytes for two inner dimensions per lane half, four per k-step (half h takes
// d = 4p + 2h and 4p + 2h + 1), while the chunk_d kernel reads such rows whole (JPF = 32).
// Both operands are rows of tables in LDS selected by a code byte: the A thermometer table
// (row = THERMO code) and the stream table (row = B code), so the inner loop is LDS reads
// and MFMAs.
//
// Two kernels:
//  * sc_gemm_fp4_kernel — persistent and balanced. The work is the list of (tile, group of
//    8 inner dimensions) pairs, tile-major; workgroup c takes the contiguous range
//    [c*W/G, (c+1)*W/G) of W pairs, G = grid size, so every workgroup gets the same work
//    whether or not the tile count divides the CU count. A tile whose groups are shared
//    by several workgroups is finished by the last one to arrive: each contributor
//    stores its exact partial sums to a workspace slot, then bumps the tile's counter;
//    the one that sees the final count adds the others' slots and applies the epilogue.
//    Nobody waits for anybody, so every workgroup runs to completion unconditionally.
//  * sc_gemm_fp4_chunked_kernel — chunk_d: per-chunk fp32 epilogue summed in chunk
//    order inside one workgroup (order-dependent, so never split across workgroups).
//
// This header holds the kernel templates; gemm_fp4_jp{32,64,128,256}.hip instantiate them
// for one table width each (separate translation units compile in parallel).
#pragma once

#include <type_traits>
#include "gemm_common.h"

namespace scmp {

__device__ __forceinline__ v16f mfma_fp4(v4i a, v4i b, v16f c) {
    v8i A = {a.x, a.y, a.z, a.w, 0, 0, 0, 0};
    v8i B = {b.x, b.y, b.z, b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, B, c, 4, 4, 0, 0, 0, 0);
}

// Where the stream tables live: one table in LDS, every class table in LDS (per-d
// classes, when they fit), per-class tables read from global memory, or one class table
// at a time in LDS, replaced where the class of the 8-d groups changes (inner dimensions
// laid out in runs of one class).
enum { LUT_LDS = 0, LUT_LDS_CLASSES = 1, LUT_GLOBAL = 2, LUT_RUNS = 3 };

// floats of the per-tile epilogue area: 3 factors per row and per column, then one int64
// output offset per row (two floats' worth each), for the largest tile shapes: 256 x 256
// (2048 floats) and 128 x 512 (2176), then the finisher flag (one int, padded to 16 bytes)
constexpr int kFactorFloats = 5 * 128 + 3 * 512 + 4;

// Tile shapes of the persistent kernel (rows of A x rows of B per workgroup, four waves):
// 256 x 256 (2 x 2 waves of 128 x 128), narrow 256 x 64 (4 x 1 waves of 64 x 64) for outputs
// at most 64 wide, wide 128 x 512 (1 x 4 waves of 128 x 128), which pads a row count
// such as 1365 to 1408 instead of 1536, and 256 x 224 (4 x 1 waves of 64 x 224) for outputs
// 193 to 224 wide (an attention head's 197 keys: 12% less padding than 256).
enum { TILE_SQUARE = 0, TILE_NARROW = 1, TILE_WIDE = 2, TILE_224 = 3 };

// accelerator complex dies (XCDs) of an MI355X; workgroup i runs on XCD i mod 8
constexpr int kXcds = 8;

template <int JPF>
struct Fp4Geom {
    static constexpr int ROWB = (JPF < 32 ? 32 : JPF) / 2;      // bytes per stored table row
    static constexpr int KS = JPF >= 64 ? JPF / 64 : 1;          // MFMA k-steps per d
    // pipeline unit: KSU k-steps of one d (two d for JPF = 32, four for 16); SPD units per d
    static constexpr int KSU = KS > 2 ? 2 : KS;
    static constexpr int SPD = KS / KSU;
    static constexpr int DPU = JPF == 16 ? 4 : JPF == 32 ? 2 : 1;    // d per unit (<= 1 k-step)
    static constexpr int UPG = JPF <= 32 ? 8 / DPU : 8 * SPD;        // units per 8 codes
    // odd number of 16-byte chunks between LDS rows: spreads rows over the bank groups;
    // JPF = 16 keeps only the 8 bytes of its 16 intervals, 8 bytes apart (every bank pair
    // holds rows, where a 16-byte stride would leave half the banks unread)
    static constexpr int LS = JPF == 16 ? 8 : 16 * ((ROWB / 16) | 1);
    static constexpr int TAB = 256 * LS;                          // one table in LDS
};

template <int JPF, int BA, int BB>
struct Fp4Frag {
    v4i a[BA][Fp4Geom<JPF>::KSU];
    v4i b[BB][Fp4Geom<JPF>::KSU];
};

// Interleave of one unit's MFMAs with the next unit's LDS reads and address arithmetic,
// front-loaded: MFMA k is followed by VPK VALU instructions until NVT
// are placed, and by DPK LDS reads from MFMA DS0 on, so the next unit's address arithmetic
// and table reads are issued in the first MFMAs of the unit and their results arrive well
// before the next unit's MFMAs need them.
template <int K, int NM, int NDS, int NVT, int VPK, int DPK, int DS0>
__device__ __forceinline__ void interleave_front() {
    if constexpr (K < NM) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
        constexpr int vd = K * VPK;
        if constexpr (vd < NVT)
            __builtin_amdgcn_sched_group_barrier(0x002, (NVT - vd) < VPK ? (NVT - vd) : VPK, 0);
        constexpr int dd = (K - DS0) * DPK;
        if constexpr (K >= DS0 && dd < NDS)
            __builtin_amdgcn_sched_group_barrier(0x100, (NDS - dd) < DPK ? (NDS - dd) : DPK, 0);
        interleave_front<K + 1, NM, NDS, NVT, VPK, DPK, DS0>();
    }
}

// The pinned schedule of one unit (NM MFMAs, NDS LDS reads of the next unit), front-loaded
// with the VALU count of each table width's unit (about 24 at JPF >= 128, 22 at 64, 52 at
// 16); the slots per MFMA were chosen by timing at cfg2 and cfg5.
template <int JPF, int NM, int NDS>
__device__ __forceinline__ void interleave_pinned() {
    if constexpr (JPF >= 128) interleave_front<0, NM, NDS, 24, 3, 1, 1>();
    else if constexpr (JPF == 64) interleave_front<0, NM, NDS, 22, 4, 2, 2>();
    else interleave_front<0, NM, NDS, 52, 8, 2, 1>();
}

// LDS layout of both kernels: the thermometer table is a static array (its address is a
// compile-time constant, so a lookup's address is its scaled code with the base in the
// read's offset field), then the dynamic area [stream table(s) | epilogue factors].
// Bytes of the stream tables in the dynamic area:
template <int JPF, int LUTSRC>
__device__ __forceinline__ int fp4_tables_bytes(const GemmP &P) {
    using G = Fp4Geom<JPF>;
    return G::TAB * (LUTSRC == LUT_LDS || LUTSRC == LUT_RUNS ? 1
                     : LUTSRC == LUT_LDS_CLASSES                ? P.nclass
                                                                : 0);
}

// Copies `rows` stored table rows (ROWB bytes apart) into LDS rows LS bytes apart.
template <int JPF>
__device__ __forceinline__ void fp4_copy_rows(uint8_t *dst, const uint8_t *src, int rows, int tid,
                                              int nt) {
    using G = Fp4Geom<JPF>;
    if constexpr (JPF == 16) {
        for (int r = tid; r < rows; r += nt)
            *(uint2 *)(dst + r * G::LS) = *(const uint2 *)(src + (int64_t)r * G::ROWB);
    } else {
        constexpr int CH = G::ROWB / 16;         // 16-byte chunks per row
        const v4i *s = (const v4i *)src;
        for (int e = tid; e < rows * CH; e += nt) {
            const int row = e / CH, col = e - row * CH;
            *(v4i *)(dst + row * G::LS + 16 * col) = s[e];
        }
    }
}

// Prologue: the thermometer table T[code][j'] = sign(code) if j' < j(code) else 0 (rows =
// THERMO code byte: bipolar sign bit | j, unipolar j), and the stream table(s) copied in
// (LUT_RUNS: by the accumulation loop, per run).
template <int JPF, int LUTSRC, int NT>
__device__ __forceinline__ void fp4_load_tables(const GemmP &P, uint8_t *sA, uint8_t *sB) {
    using G = Fp4Geom<JPF>;
    constexpr int U = G::ROWB / 4;             // dwords per stored row (8 intervals each)
    constexpr int UL = G::LS / 4 < U ? G::LS / 4 : U;   // of them kept in LDS
    const int Ut = P.JP < 8 * U ? P.JP / 8 : U; // dwords holding intervals (JP = 16: 2)
    const int tid = threadIdx.x;
    for (int e = tid; e < 256 * UL; e += NT) {
        const int row = e / UL, u = e - row * UL;
        const int j = P.bipolar ? (row & 0x7f) : row;
        const uint32_t one = (P.bipolar && (row & 0x80)) ? 0xAu : 0x2u;
        uint32_t w = 0;
        if (u < Ut) {
#pragma unroll
            for (int b = 0; b < 8; ++b)
                if (8 * u + b < j) w |= one << (4 * b);
        }
        *(uint32_t *)(sA + row * G::LS + 4 * u) = w;
    }
    if (LUTSRC == LUT_LDS || LUTSRC == LUT_LDS_CLASSES)
        fp4_copy_rows<JPF>(sB, (const uint8_t *)P.lut,
                           (LUTSRC == LUT_LDS_CLASSES ? P.nclass : 1) * 256, tid, NT);
}

// acc += the products of inner-dimension groups [g0, g1) (8 d per group) for the operand
// rows of the wave's A blocks (BA blocks of 32 rows from the wave-uniform address abase,
// row stride lda) and B blocks (BB from bbase, stride ldb); the lane's row li of each block
// is addressed by a 32-bit offset from that scalar base. Each pipeline unit
// (up to two k-steps of one d, or two d for JPF = 32) is loaded one unit ahead into the
// other of two fragment sets, so the LDS reads of unit u+1 overlap the MFMAs of unit u.
// Code bytes: the A side loads one uint2 per row and group into one of two buffers that
// alternate by group parity (group g+2's codes are issued when group g ends); the B side
// loads one 16-byte pair of groups (gp, gp+1) per row, half the load instructions and
// cache-line requests of one load per group, and the pair after next is issued when a
// pair ends. Either way a load is read two groups after it is issued, and no wait covers a
// load issued in the same group. A pair load never reads past a code row: its address is
// clamped to the row's last two groups (the pair's first group then sits in the upper
// half, `shift` 1; only a segment's lone last group can be so). after(d0, d1) runs once
// the MFMAs of inner dimensions d0..d1 are all issued.
template <int JPF, int BA, int BB, int LUTSRC, bool SCHED, class After>
__device__ __forceinline__ void fp4_accumulate(const GemmP &P, const uint8_t *sA,
                                               const uint8_t *sB, const uint8_t *abase,
                                               const uint8_t *bbase, int li, int g0, int g1,
                                               int h, v16f (&acc)[BA][BB], After after) {
    using G = Fp4Geom<JPF>;
    constexpr int ROWB = G::ROWB, KSU = G::KSU, SPD = G::SPD, UPG = G::UPG, LS = G::LS,
                  TAB = G::TAB;
    constexpr int NR = BA + BB;                  // code rows per lane: A rows, then B rows
    constexpr bool PERD = LUTSRC == LUT_LDS_CLASSES || LUTSRC == LUT_GLOBAL;   // per-d classes
    const uint8_t *glut = (const uint8_t *)P.lut;
    const int D = P.D;
    const int ngroups = (D + 7) / 8;
    const int glast = ngroups >= 2 ? ngroups - 2 : 0;   // last pair address (in groups)

    // With per-d table classes, lane l also loads the class of inner dimension 8g + (l & 7)
    // of each group into cls.x; a unit takes its d's class from that lane (v_readlane), so
    // the class costs no memory wait inside the loop. JPF = 16: each lane loads the classes
    // of the four inner dimensions its lane half takes in the group's two units (cls.x, .y:
    // d = 8g + 2h, +1; cls.z, .w: d = 8g + 4 + 2h, +1), so a unit's table bases need no
    // cross-lane moves.
    const int lane8 = (int)(threadIdx.x & 7);
    // lane offsets of row li of block 0 (a block is 32 rows further); all below 2^31, as
    // the host bounds D (and so the row strides) by 65536
    const uint32_t lda = (uint32_t)P.lda, ldb = (uint32_t)P.ldb;
    const uint32_t oa = (uint32_t)li * lda, ob = (uint32_t)li * ldb;
    auto load_a = [&](uint2 (&c)[BA], int4 &cls, int g) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BA; ++i)
            c[i] = *(const uint2 *)(abase + (oa + 32u * (uint32_t)i * lda + 8u * (uint32_t)g));
        if (PERD) {
            // an unconditional load (the index clamped to the last d; classes past D meet
            // zero codes): a load under a branch makes the compiler wait for every load in
            // flight, the code prefetches included, before the next one
            if constexpr (JPF == 16) {
                // 32-bit indices: scalar base + vector offset addressing
                const uint32_t dmax = (uint32_t)D - 1u;
                const uint32_t d0 = 8u * (uint32_t)g + 2u * (uint32_t)h;
                cls.x = P.d_class[d0 < dmax ? d0 : dmax];
                cls.y = P.d_class[d0 + 1u < dmax ? d0 + 1u : dmax];
                cls.z = P.d_class[d0 + 4u < dmax ? d0 + 4u : dmax];
                cls.w = P.d_class[d0 + 5u < dmax ? d0 + 5u : dmax];
            } else {
                const int d = 8 * g + lane8;
                cls.x = P.d_class[d < D ? d : D - 1];
            }
        }
        if (LUTSRC == LUT_RUNS) {
            // the group's class, by a vector load issued after the codes: waiting for it
            // waits for nothing that is not needed at the same point
            int z = 0;
            asm volatile("" : "+v"(z));
            cls.x = P.group_class[g + z];
        }
    };
    // a pair starts at an odd group as often as at an even one: 8-byte aligned 16-byte loads
    struct __attribute__((aligned(8))) pair_t {
        uint32_t x, y, z, w;
    };
    auto load_b = [&](uint4 (&q)[BB], int gp) __attribute__((always_inline)) {
        const int gl = gp < glast ? gp : glast;
#pragma unroll
        for (int j = 0; j < BB; ++j) {
            const pair_t t =
                *(const pair_t *)(bbase + (ob + 32u * (uint32_t)j * ldb + 8u * (uint32_t)gl));
            q[j] = make_uint4(t.x, t.y, t.z, t.w);
        }
    };
    auto shift_of = [&](int gp) __attribute__((always_inline)) {
        return gp - (gp < glast ? gp : glast);
    };
    // code byte of inner dimension dl (0..7, a compile-time constant): A row i of a group,
    // or B row j of half m (0: first group of the pair, 1: second)
    auto code_a = [](const uint2 (&c)[BA], int i, int dl) __attribute__((always_inline)) {
        return (int)(((dl < 4 ? c[i].x : c[i].y) >> (8 * (dl & 3))) & 0xffu);
    };
    auto code_b = [](const uint4 (&q)[BB], int m, int j, int dl) __attribute__((always_inline)) {
        const uint32_t w = dl < 4 ? (m ? q[j].z : q[j].x) : (m ? q[j].w : q[j].y);
        return (int)((w >> (8 * (dl & 3))) & 0xffu);
    };
    // JPF <= 32: the lane half h selects which code bytes of a word it takes. Rotating the
    // word right by `rot` bits moves them to fixed byte positions, so a lookup costs a
    // constant-position byte extract instead of a variable shift; word w of row i (w = 0, 1:
    // the group's d 0-3, 4-7), byte t after the rotation. JPF = 16 rotates by 24 - 16h, which
    // puts the half's bytes 2h, 2h + 1 at positions 1 and 2: a byte there is extracted and
    // scaled to a row offset by one instruction (a shift with a byte-select operand); JPF = 32
    // rotates by 8h.
    const uint32_t rot = JPF == 16 ? 24u - 16u * (uint32_t)h : 8u * (uint32_t)h;
    auto rbyte = [&](uint32_t w, int t) __attribute__((always_inline)) {
        return (int)((__builtin_amdgcn_alignbit(w, w, rot) >> (8 * t)) & 0xffu);
    };
    auto rcode_a = [&](const uint2 (&c)[BA], int i, int w, int t) __attribute__((always_inline)) {
        return rbyte(w ? c[i].y : c[i].x, t);
    };
    auto rcode_b = [&](const uint4 (&q)[BB], int m, int j, int w, int t)
        __attribute__((always_inline)) {
        return rbyte(w ? (m ? q[j].w : q[j].y) : (m ? q[j].z : q[j].x), t);
    };

    // JPF = 16: the lane half's two inner dimensions dl, dl + 1 of a unit, 8 bytes (16
    // intervals) of a table row each, side by side in one fragment
    auto stage16 = [&](Fp4Frag<JPF, BA, BB> &F, const uint2 (&ca)[BA], int4 cls4,
                       const uint4 (&qb)[BB], int m, int unit) __attribute__((always_inline)) {
        // d 4 unit + 2h and + 1: bytes 1 and 2 of word `unit` rotated by 24 - 16h
#pragma unroll
        for (int i = 0; i < BA; ++i) {
            const uint2 r0 = *(const uint2 *)(sA + rcode_a(ca, i, unit, 1) * LS);
            const uint2 r1 = *(const uint2 *)(sA + rcode_a(ca, i, unit, 2) * LS);
            F.a[i][0] = (v4i){(int)r0.x, (int)r0.y, (int)r1.x, (int)r1.y};
        }
        const uint8_t *base0 = sB, *base1 = sB;
        if (PERD) {
            const int k0 = unit ? cls4.z : cls4.x, k1 = unit ? cls4.w : cls4.y;
            base0 = LUTSRC == LUT_GLOBAL ? glut + (int64_t)k0 * 256 * ROWB : sB + k0 * TAB;
            base1 = LUTSRC == LUT_GLOBAL ? glut + (int64_t)k1 * 256 * ROWB : sB + k1 * TAB;
        }
        constexpr int RS = LUTSRC == LUT_GLOBAL ? ROWB : LS;
#pragma unroll
        for (int j = 0; j < BB; ++j) {
            const uint2 r0 = *(const uint2 *)(base0 + rcode_b(qb, m, j, unit, 1) * RS);
            const uint2 r1 = *(const uint2 *)(base1 + rcode_b(qb, m, j, unit, 2) * RS);
            F.b[j][0] = (v4i){(int)r0.x, (int)r0.y, (int)r1.x, (int)r1.y};
        }
    };
    // load unit `unit` of the group whose first d is dg (A codes ca, B codes: half m of qb)
    auto stage = [&](Fp4Frag<JPF, BA, BB> &F, const uint2 (&ca)[BA], int4 cls4,
                     const uint4 (&qb)[BB], int m, int unit, int dg)
        __attribute__((always_inline)) {
        if constexpr (JPF == 16) {
            stage16(F, ca, cls4, qb, m, unit);
            return;
        }
        const int dl = JPF == 32 ? 2 * unit + h : unit / SPD;    // d within the group
        const int koff = (JPF == 32 ? 0 : 16 * h) + 32 * KSU * (unit % SPD);
        // JPF = 32: d 2 unit + h is byte 2 (unit & 1) of word unit / 2 rotated by 8h
        const int w32 = unit >> 1, t32 = 2 * (unit & 1);
#pragma unroll
        for (int i = 0; i < BA; ++i) {
            const int code = JPF == 32 ? rcode_a(ca, i, w32, t32) : code_a(ca, i, dl);
            const uint8_t *p = sA + code * LS + koff;
#pragma unroll
            for (int t = 0; t < KSU; ++t) F.a[i][t] = *(const v4i *)(p + 32 * t);
        }
        const uint8_t *base = sB;
        if (PERD) {
            int cls;
            if (JPF == 32) {                     // the lane halves take d = 2 unit + h
                const int c0 = __builtin_amdgcn_readlane(cls4.x, 2 * unit);
                const int c1 = __builtin_amdgcn_readlane(cls4.x, 2 * unit + 1);
                cls = h ? c1 : c0;
            } else {
                cls = __builtin_amdgcn_readlane(cls4.x, unit / SPD);
            }
            base = LUTSRC == LUT_GLOBAL ? glut + (int64_t)cls * 256 * ROWB : sB + cls * TAB;
        }
#pragma unroll
        for (int j = 0; j < BB; ++j) {
            const int code = JPF == 32 ? rcode_b(qb, m, j, w32, t32) : code_b(qb, m, j, dl);
            const uint8_t *p = base + code * (LUTSRC == LUT_GLOBAL ? ROWB : LS) + koff;
#pragma unroll
            for (int t = 0; t < KSU; ++t) F.b[j][t] = *(const v4i *)(p + 32 * t);
        }
    };
    auto done = [&](int unit, int dg) __attribute__((always_inline)) {
        if (unit % SPD != SPD - 1) return;
        if (JPF <= 32) after(dg + G::DPU * unit, dg + G::DPU * unit + G::DPU - 1);
        else after(dg + unit / SPD, dg + unit / SPD);
    };
    auto mma = [&](const Fp4Frag<JPF, BA, BB> &F) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < KSU; ++t)
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int j = 0; j < BB; ++j) acc[i][j] = mfma_fp4(F.a[i][t], F.b[j][t], acc[i][j]);
    };

    // LUT_RUNS: the table of class c (clamped to the valid classes) replaces the one in LDS
    // once every wave is done reading it; the whole workgroup runs the same groups, so every
    // wave reaches the same barriers
    auto run_table = [&](int c) __attribute__((always_inline)) {
        c = c < 0 ? 0 : c >= P.nclass ? P.nclass - 1 : c;
        __syncthreads();
        fp4_copy_rows<JPF>((uint8_t *)sB, glut + (int64_t)c * 256 * ROWB, 256,
                           (int)threadIdx.x, (int)blockDim.x);
        __syncthreads();
    };

    Fp4Frag<JPF, BA, BB> F0, F1;
    // one group g (A codes ca, B codes half m of qb); its last unit stages unit 0 of the
    // next group (A codes can, B codes half mn of qbn), then runs `refill`
    auto group = [&](const uint2 (&ca)[BA], int4 cls, const uint4 (&qb)[BB], int m, int g,
                     const uint2 (&can)[BA], int4 clsn, const uint4 (&qbn)[BB], int mn,
                     auto refill) __attribute__((always_inline)) {
        const int dg = 8 * g;
#pragma unroll
        for (int uu = 0; uu < UPG; uu += 2) {
            stage(F1, ca, cls, qb, m, uu + 1, dg);
            mma(F0);
            if (SCHED) {
                interleave_pinned<JPF, BA * BB * KSU, NR * KSU * (JPF == 16 ? 2 : 1)>();
                __builtin_amdgcn_sched_barrier(0);
            }
            done(uu, dg);
            if (uu + 2 < UPG) {
                stage(F0, ca, cls, qb, m, uu + 2, dg);
            } else {
                if (LUTSRC == LUT_RUNS) {
                    const int cn = __builtin_amdgcn_readfirstlane(clsn.x);
                    if (cn != __builtin_amdgcn_readfirstlane(cls.x)) run_table(cn);
                }
                stage(F0, can, clsn, qbn, mn, 0, dg + 8);
                refill();
            }
            mma(F1);
            if (SCHED) {
                interleave_pinned<JPF, BA * BB * KSU, NR * KSU * (JPF == 16 ? 2 : 1)>();
                __builtin_amdgcn_sched_barrier(0);
            }
            done(uu + 1, dg);
        }
    };

    // A: a0 / a1 hold groups of even / odd offset from g0; B: qc holds the pair (g, g+1),
    // qn the pair (g+2, g+3), in flight
    uint2 a0[BA], a1[BA];
    uint4 qc[BB], qn[BB];
    int4 cl0 = {0, 0, 0, 0}, cl1 = {0, 0, 0, 0};
    load_a(a0, cl0, g0);
    load_a(a1, cl1, g0 + 1 < g1 ? g0 + 1 : g1 - 1);
    load_b(qc, g0);
    load_b(qn, g0 + 2);
    int sc = shift_of(g0);                       // 1 only for a lone last group
    if (LUTSRC == LUT_RUNS) run_table(__builtin_amdgcn_readfirstlane(cl0.x));
    stage(F0, a0, cl0, qc, sc, 0, 8 * g0);
    int g = g0;
    // full pairs: g + 1 < g1 <= ngroups, so qc's shift is 0; the loop body has no branch
    for (; g + 1 < g1; g += 2) {
        const int sn = shift_of(g + 2);
        group(a0, cl0, qc, 0, g, a1, cl1, qc, 1,
              [&] { load_a(a0, cl0, g + 2 < g1 ? g + 2 : g1 - 1); });
        group(a1, cl1, qc, 1, g + 1, a0, cl0, qn, sn, [&] {
            load_a(a1, cl1, g + 3 < g1 ? g + 3 : g1 - 1);
#pragma unroll
            for (int j = 0; j < BB; ++j) qc[j] = qn[j];
            sc = sn;
            load_b(qn, g + 4 < g1 ? g + 4 : g1 - 1);
        });
    }
    // a lone last group: A codes in a0, B codes half sc of qc (the unit staged for it at the
    // end of the previous pair used the same half)
    if (g < g1) group(a0, cl0, qc, sc, g, a1, cl1, qn, 0, [] {});
}

// Balanced schedule: workgroup c of nwg owns work items [first(c), first(c+1)) of W.
__device__ __forceinline__ int64_t sched_first(int64_t c, int64_t W, int64_t nwg) {
    return c * W / nwg;
}
// The workgroup that owns work item u: the largest c with first(c) <= u.
__device__ __forceinline__ int64_t sched_owner(int64_t u, int64_t W, int64_t nwg) {
    return ((u + 1) * nwg - 1) / W;
}
// Partial-sum slot of workgroup c for tile t: 2c for its first segment, 2c + 1 for its
// last one (a workgroup's range touches at most two shared tiles).
__device__ __forceinline__ int64_t fp4_slot(int64_t c, int64_t t, int64_t W, int64_t nwg,
                                            int ngroups) {
    return 2 * c + (sched_first(c, W, nwg) / ngroups == t ? 0 : 1);
}

// Per-wave staging area of the drain: one 32 x 32 block, rows kStageStride floats apart (the
// two lane halves' rows, 4 apart, then fall on disjoint bank halves).
constexpr int kStageStride = 40;
constexpr int kStageFloats = 32 * kStageStride;          // per wave

// four floats at a 4-byte aligned address (rows whose stride is not a multiple of 4
// floats): one 16-byte store
struct __attribute__((aligned(4))) f4u {
    float x, y, z, w;
};

// Fused epilogue of a finished tile. In the MFMA layout lane (li, h) of block (i, c) holds
// row 32i + 8(r>>2) + 4h + (r&3) and column 32c + li of the wave's quadrant; the epilogue is
// applied there (row factors and output row offsets from LDS, column factors once per block
// column), each block's values go through the wave's staging area in LDS, and lane L reads
// back 4 consecutive columns 4(L & 7).. of rows (L >> 3) + 8k, so the tile leaves as 16-byte
// stores (a quarter of the store instructions of one float per lane, which measured the
// drain's bound); a group of columns that runs past M is stored value by value. Only
// stores reach global memory (any load between them would make the wave wait for every
// earlier store on gfx9).
template <int KIND, int BA, int BB, int TR, int TC>
__device__ __forceinline__ void fp4_drain(const GemmP &P, const v16f (&acc)[BA][BB],
                                          const float *s_rowf, const float *s_colf,
                                          const int64_t *s_rowo, const EpiUniform &eu,
                                          float *stg, int lane, int nrw, int mcw, int tc0,
                                          int64_t ybase) {
    const int h = lane >> 5, li = lane & 31;
    const int rq = lane >> 3, cq = 4 * (lane & 7);
    float cb[BB], cz[BB], cs[BB];
#pragma unroll
    for (int c = 0; c < BB; ++c) {
        const int mc = mcw + 32 * c + li;
        cb[c] = s_colf[mc];
        cz[c] = s_colf[TC + mc];
        cs[c] = s_colf[2 * TC + mc];
    }
    constexpr bool ZP = KIND == SCMP_EPI_ZP_ROWCOL || KIND == SCMP_EPI_ZP_SCALAR;
    constexpr bool RA = KIND == SCMP_EPI_ROWCOL || KIND == SCMP_EPI_ZP_ROWCOL;
#pragma unroll
    for (int i = 0; i < BA; ++i) {
        float ra[16], rz[16], rs[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int nr = nrw + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
            ra[r] = RA ? s_rowf[nr] : 0.f;
            rz[r] = KIND == SCMP_EPI_ZP_ROWCOL ? s_rowf[TR + nr] : 0.f;
            rs[r] = ZP ? s_rowf[2 * TR + nr] : 0.f;
        }
        int64_t ro[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) ro[k] = s_rowo[nrw + 32 * i + rq + 8 * k];
#pragma unroll
        for (int c = 0; c < BB; ++c) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float v = KIND == SCMP_EPI_INT
                                    ? __int_as_float((int32_t)acc[i][c][r])
                                    : epilogue_apply_k<KIND>(P.epi, acc[i][c][r], ra[r], rz[r],
                                                             rs[r], cb[c], cz[c], cs[c], eu);
                stg[(8 * (r >> 2) + 4 * h + (r & 3)) * kStageStride + li] = v;
            }
            const int m = tc0 + mcw + 32 * c + cq;
            const int nv = P.M - m;                           // valid columns from m
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const v4f v = *(const v4f *)(stg + (rq + 8 * k) * kStageStride + cq);
                if (ro[k] < 0 || nv <= 0) continue;           // row past N, columns past M
                const int64_t o = ybase + ro[k] + m;
                if (nv >= 4) {
                    if constexpr (KIND == SCMP_EPI_INT)
                        *(f4u *)(P.iout + o) = f4u{v[0], v[1], v[2], v[3]};
                    else
                        *(f4u *)(P.y + o) = f4u{v[0], v[1], v[2], v[3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 3; ++e) {
                        if (e >= nv) break;
                        if constexpr (KIND == SCMP_EPI_INT)
                            P.iout[o + e] = __float_as_int(v[e]);
                        else
                            P.y[o + e] = v[e];
                    }
                }
            }
        }
    }
}

template <int JPF, int BA, int BB, int WA, int WB, int LUTSRC, bool SCHED>
__global__ void __launch_bounds__(64 * WA * WB)
sc_gemm_fp4_kernel(GemmP P) {
    constexpr int NT = 64 * WA * WB;
    constexpr int NW = WA * WB;
    constexpr int TILE_FLOATS = NW * BA * BB * 1024;   // accumulators of one tile
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ __attribute__((aligned(16))) uint8_t sA[Fp4Geom<JPF>::TAB];  // thermometer
    const int tabs = fp4_tables_bytes<JPF, LUTSRC>(P);
    uint8_t *sB = smem;                                  // stream table(s)
    constexpr int TR = WA * BA * 32, TC = WB * BB * 32;   // tile rows / columns
    static_assert(5 * TR + 3 * TC + 1 <= kFactorFloats, "epilogue factor area too small");
    float *s_rowf = (float *)(smem + ((tabs + 15) & ~15)); // [3][TR] sa, za, suma
    float *s_colf = s_rowf + 3 * TR;                     // [3][TC] sb, zb, sumb
    int64_t *s_rowo = (int64_t *)(s_colf + 3 * TC);      // [TR] output row offsets
    // the finisher flag lives in the dynamic area too: with no static LDS the tables start
    // at LDS address 0, and a table row's address is its scaled code alone
    int &s_last = *(int *)(s_rowo + TR);
    float *s_stage = s_rowf + kFactorFloats;             // [NW][kStageFloats] drain staging

    fp4_load_tables<JPF, LUTSRC, NT>(P, sA, sB);
    __syncthreads();

    const int tid = threadIdx.x;
    // wave index as a scalar: every per-wave offset (partial-sum blocks, staging area,
    // operand rows) then lives in scalar registers instead of one vector register each
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, li = lane & 31;
    const int wa = wave % WA, wb = wave / WA;
    const int ngroups = (P.D + 7) / 8;
    const int64_t tiles_per_batch = (int64_t)P.tilesA * P.tilesB;
    const int64_t W = P.ntiles * ngroups;
    const int64_t nwg = gridDim.x;
    // Workgroups are dispatched round-robin over the XCDs; number the workers so that
    // consecutive ranges (the ones sharing a tile) run on the same XCD and its L2.
    const int64_t c_self = nwg % kXcds == 0
                               ? (blockIdx.x % kXcds) * (nwg / kXcds) + blockIdx.x / kXcds
                               : (int64_t)blockIdx.x;
    const int64_t u_end = sched_first(c_self + 1, W, nwg);
    // work lists below 2^31 items (every practical launch) index tiles in 32-bit arithmetic
    const bool w32 = W < ((int64_t)1 << 31);

    for (int64_t u = sched_first(c_self, W, nwg); u < u_end;) {
        int64_t t, batch;
        int g0, ta, tb;
        if (w32) {
            const uint32_t ng = (uint32_t)ngroups, t32 = (uint32_t)u / ng;
            const uint32_t tpb = (uint32_t)tiles_per_batch, b32 = t32 / tpb;
            const uint32_t rem = t32 - b32 * tpb, tA = (uint32_t)P.tilesA;
            t = t32;
            batch = b32;
            g0 = (int)((uint32_t)u - t32 * ng);
            ta = (int)(rem % tA);
            tb = (int)(rem / tA);
        } else {
            t = u / ngroups;
            g0 = (int)(u - t * ngroups);
            batch = t / tiles_per_batch;
            const int64_t rem = t - batch * tiles_per_batch;
            ta = (int)(rem % P.tilesA);
            tb = (int)(rem / P.tilesA);
        }
        const int g1 = (int)(u_end - t * ngroups < ngroups ? u_end - t * ngroups : ngroups);
        const int a0 = (ta * WA + wa) * (BA * 32);
        const int b0 = (tb * WB + wb) * (BB * 32);

        // wave-uniform bases of the wave's first A and B rows
        const uint8_t *abase = P.ca + batch * P.bsa + (int64_t)a0 * P.lda;
        const uint8_t *bbase = P.cb + batch * P.bsb + (int64_t)b0 * P.ldb;

        v16f acc[BA][BB];
#pragma unroll
        for (int i = 0; i < BA; ++i)
#pragma unroll
            for (int c = 0; c < BB; ++c) acc[i][c] = (v16f){0.0f};
        // the tile-uniform epilogue values (the head's scales of a per-head product), loaded
        // now so that their latency passes under the first code loads, not at the drain
        const bool fp32 = P.epi.kind != SCMP_EPI_INT;
        const EpiUniform eu = fp32 ? epi_uniform(P.epi, batch) : EpiUniform{0.f, 0.f, 0.f, 0.f};
        fp4_accumulate<JPF, BA, BB, LUTSRC, SCHED>(P, sA, sB, abase, bbase, li, g0, g1, h, acc,
                                                    [](int, int) {});

        // The lane index, re-read inside the tile loop through an opaque copy: offsets
        // derived from it are then computed here, when needed, instead of being hoisted
        // out of the loop into registers that the main loop's pressure would spill.
        int lt = lane;
        asm volatile("" : "+v"(lt));
        // partial-sum slot layout: block (i, c) of this wave, then the quarter q of the
        // lane's 16 accumulator registers, then lane (4 floats each): one 16-byte access per
        // lane covers 1 KB of consecutive memory
        auto pofs = [&](int i, int c, int q) __attribute__((always_inline)) {
            return (int64_t)((wave * BA + i) * BB + c) * 1024 + q * 256 + lt * 4;
        };

        const bool shared = g0 != 0 || g1 != ngroups;
        bool finish = true;
        int64_t cf = 0, cl = -1;
        if (shared) {
            // A tile shared with other workgroups: publish this workgroup's partial sums
            // (slot 0: its first segment, slot 1: its last one) straight from the
            // accumulators, then count in; the workgroup that completes the count
            // finishes the tile.
            const int64_t tfirst = t * ngroups;
            cf = sched_owner(tfirst, W, nwg);
            cl = sched_owner(tfirst + ngroups - 1, W, nwg);
            float *mine = P.part + fp4_slot(c_self, t, W, nwg, ngroups) * (int64_t)TILE_FLOATS;
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int c = 0; c < BB; ++c) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *(v4f *)(mine + pofs(i, c, q)) =
                            (v4f){acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2],
                                  acc[i][c][4 * q + 3]};
                }
            // Deferred: the fixup launch that follows this one finishes the tile (the
            // kernel boundary orders the stores before its loads).
            if (P.deferred) {
                u = t * ngroups + g1;
                continue;
            }
            // The barrier waits for every wave's stores; one device-scope fence then
            // publishes them (and, for the finisher, makes the others' visible: the L1
            // and L2 invalidation it performs covers the whole CU).
            __syncthreads();
            if (tid == 0) {
                __threadfence();
                const int seen = atomicAdd(&P.cnt[t], 1);
                const int last = seen == (int)(cl - cf);
                if (last) {
                    P.cnt[t] = 0;                    // ready for the next launch
                    __threadfence();
                }
                s_last = last;
            }
            __syncthreads();
            finish = s_last != 0;
            if (finish) {
                // add the other contributors' exact partial sums into the accumulators
                // (integers below 2^24: exact in any order), all loads of a row of
                // blocks issued before their adds
                for (int64_t c2 = cf; c2 <= cl; ++c2) {
                    if (c2 == c_self) continue;
                    const float *other =
                        P.part + fp4_slot(c2, t, W, nwg, ngroups) * (int64_t)TILE_FLOATS;
#pragma unroll
                    for (int i = 0; i < BA; ++i) {
                        v4f ov[BB][4];
#pragma unroll
                        for (int c = 0; c < BB; ++c)
#pragma unroll
                            for (int q = 0; q < 4; ++q)
                                ov[c][q] = __builtin_nontemporal_load(
                                    (const v4f *)(other + pofs(i, c, q)));
#pragma unroll
                        for (int c = 0; c < BB; ++c)
#pragma unroll
                            for (int q = 0; q < 4; ++q)
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[i][c][4 * q + e] += ov[c][q][e];
                    }
                }
            }
        }

        if (finish) {
            // the tile's epilogue factors, once: row factors of its TR rows and column
            // factors of its TC columns into LDS, the uniform ones into registers
            const int tr0 = ta * TR, tc0 = tb * TC;
            __syncthreads();          // every wave is past the previous tile's last store
            // where each row of the tile goes (row map applied, times ldy; -1 past N): the
            // drain below then issues no loads, so no store ever waits for another
            for (int e = tid; e < TR; e += NT)
                s_rowo[e] = tr0 + e < P.N ? out_row(P.row_map, tr0 + e) * P.ldy : (int64_t)-1;
            if (fp32) {
                for (int e = tid; e < TR; e += NT) {
                    float f[3] = {0.f, 0.f, 0.f};
                    if (tr0 + e < P.N) epi_row_factors(P.epi, tr0 + e, batch, f);
                    s_rowf[e] = f[0];
                    s_rowf[TR + e] = f[1];
                    s_rowf[2 * TR + e] = f[2];
                }
                for (int e = tid; e < TC; e += NT) {
                    float f[3] = {0.f, 0.f, 0.f};
                    if (tc0 + e < P.M) epi_col_factors(P.epi, tc0 + e, batch, f);
                    s_colf[e] = f[0];
                    s_colf[TC + e] = f[1];
                    s_colf[2 * TC + e] = f[2];
                }
            }
            __syncthreads();
            const int nrw = wa * (BA * 32), mcw = wb * (BB * 32);
            float *stg = s_stage + wave * kStageFloats;
            const int64_t ybase = batch * P.bsy;
            switch (P.epi.kind) {
            case SCMP_EPI_INT:
                fp4_drain<SCMP_EPI_INT, BA, BB, TR, TC>(P, acc, s_rowf, s_colf, s_rowo, eu, stg, lt, nrw, mcw, tc0, ybase);
                break;
            case SCMP_EPI_ROWCOL:
                fp4_drain<SCMP_EPI_ROWCOL, BA, BB, TR, TC>(P, acc, s_rowf, s_colf, s_rowo, eu, stg, lt, nrw, mcw, tc0, ybase);
                break;
            case SCMP_EPI_SCALAR:
                fp4_drain<SCMP_EPI_SCALAR, BA, BB, TR, TC>(P, acc, s_rowf, s_colf, s_rowo, eu, stg, lt, nrw, mcw, tc0, ybase);
                break;
            case SCMP_EPI_HEAD:
                fp4_drain<SCMP_EPI_HEAD, BA, BB, TR, TC>(P, acc, s_rowf, s_colf, s_rowo, eu, stg, lt, nrw, mcw, tc0, ybase);
                break;
            case SCMP_EPI_ZP_ROWCOL:
                fp4_drain<SCMP_EPI_ZP_ROWCOL, BA, BB, TR, TC>(P, acc, s_rowf, s_colf, s_rowo, eu, stg, lt, nrw, mcw, tc0, ybase);
                break;
            default:
                fp4_drain<SCMP_EPI_ZP_SCALAR, BA, BB, TR, TC>(P, acc, s_rowf, s_colf, s_rowo, eu, stg, lt, nrw, mcw, tc0, ybase);
                break;
            }
        }
        u = t * ngroups + g1;
    }
}

// Deferred split tiles (P.deferred): after the persistent launch, workgroup (t, blk) of
// this launch finishes block blk of tile t when the tile was shared (its contributors are
// the workgroups whose shares of the work list overlap it; a tile that one workgroup did
// whole was drained by that workgroup). Block blk is the 32 x 32 block (i, cb) of wave w in
// the persistent kernel's partial-sum slot layout; thread tid holds its quarter q = tid / 64
// and lane, 4 values: the sum over the contributors' slots (exact integers), then the
// epilogue, stored like the fused drain. Deferred launches have fewer tiles than
// workgroups, so every schedule quantity fits 32 bits (W < 256 tiles x 8192 groups).
template <int KIND, int BA, int BB, int WA, int WB>
__global__ void __launch_bounds__(256) sc_gemm_fp4_fixup_kernel(GemmP P) {
    constexpr int NW = WA * WB, TILE_FLOATS = NW * BA * BB * 1024;
    constexpr int TR = WA * BA * 32, TC = WB * BB * 32;
    const uint32_t ngroups = (uint32_t)(P.D + 7) / 8, nwg = (uint32_t)P.nwg;
    const uint32_t W = (uint32_t)P.ntiles * ngroups;
    const uint32_t t = blockIdx.x, tg = t * ngroups;
    const uint32_t cf = ((tg + 1) * nwg - 1) / W;                   // owner of the tile start
    const uint32_t cl = ((tg + ngroups) * nwg - 1) / W;             // owner of its last group
    if (cf == cl) return;                                           // a whole tile
    // contributor cf's segment is its first one only when its share starts at the tile;
    // every later contributor's share starts inside the tile (slot 2c, as in fp4_slot)
    const uint32_t slot_cf = 2 * cf + (cf * W / nwg == tg ? 0u : 1u);
    const int blk = blockIdx.y;                         // ((w * BA + i) * BB + cb)
    const int w = blk / (BA * BB), i = (blk / BB) % BA, cb = blk % BB;
    const int tid = threadIdx.x, q = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, li = lane & 31;
    const int64_t off = (int64_t)blk * 1024 + q * 256 + lane * 4;
    const uint32_t tiles_per_batch = (uint32_t)P.tilesA * (uint32_t)P.tilesB;
    const int64_t batch = t / tiles_per_batch;
    const uint32_t rem = t - (uint32_t)batch * tiles_per_batch;
    const int ta = (int)(rem % (uint32_t)P.tilesA), tb = (int)(rem / (uint32_t)P.tilesA);
    const int wa = w % WA, wb = w / WA;
    const int mraw = tb * TC + (wb * BB + cb) * 32 + li;
    const int nb = ta * TR + (wa * BA + i) * 32 + 8 * q + 4 * h;   // rows nb .. nb + 3
    // every load issued before any is used (none under a branch: indices clamped, values
    // past N or M are computed and not stored)
    const int m = mraw < P.M ? mraw : P.M - 1;
    int64_t orow[4];
    float rf[4][3];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int n = nb + e < P.N ? nb + e : P.N - 1;
        orow[e] = out_row(P.row_map, n);
        if (KIND != SCMP_EPI_INT) epi_row_factors(P.epi, n, batch, rf[e]);
    }
    float cf3[3] = {0.f, 0.f, 0.f};
    EpiUniform eu = {0.f, 0.f, 0.f, 0.f};
    if (KIND != SCMP_EPI_INT) {
        epi_col_factors(P.epi, m, batch, cf3);
        eu = epi_uniform(P.epi, batch);
    }
    // the contributors' slots, four at a time with all four loads in flight
    constexpr int KS = 4;
    v4f sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t c0 = cf; c0 <= cl; c0 += KS) {
        v4f v[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const uint32_t c2 = c0 + k <= cl ? c0 + k : cl;
            const uint32_t slot = c2 == cf ? slot_cf : 2 * c2;
            v[k] = *(const v4f *)(P.part + (int64_t)slot * TILE_FLOATS + off);
        }
#pragma unroll
        for (int k = 0; k < KS; ++k)
            if (c0 + k <= cl) sum += v[k];              // integers below 2^24: exact
    }
    if (mraw >= P.M) return;
    const int64_t ybase = batch * P.bsy;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (nb + e >= P.N) break;
        const int64_t o = ybase + orow[e] * P.ldy + m;
        if (KIND == SCMP_EPI_INT)
            P.iout[o] = (int32_t)sum[e];
        else
            P.y[o] = epilogue_apply_k<KIND>(P.epi, sum[e], rf[e][0], rf[e][1], rf[e][2], cf3[0],
                                            cf3[1], cf3[2], eu);
    }
}

template <int JPF, int BA, int BB, int WA, int WB, int LUTSRC, bool SLDS>
__global__ void __launch_bounds__(64 * WA * WB)
sc_gemm_fp4_chunked_kernel(GemmP P) {
    constexpr int NT = 64 * WA * WB;
    constexpr int TR = WA * BA * 32, TC = WB * BB * 32;   // tile rows / columns
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ __attribute__((aligned(16))) uint8_t sA[Fp4Geom<JPF>::TAB];  // thermometer
    uint8_t *sB = smem;
    const int tid = threadIdx.x;
    const int ta = blockIdx.x % P.tilesA, tb = blockIdx.x / P.tilesA;
    const int batch = blockIdx.z;
    const int D = P.D;
    const int ngroups = (D + 7) / 8;
    const int nchunks = (D + P.chunk - 1) / P.chunk;
    const int tr0 = P.row0 + ta * TR, tc0 = tb * TC;     // the tile's first row / column
    // SLDS: every chunk's scales of the tile's rows and columns sit in LDS
    // ([chunk][TR] then [chunk][TC], zero past N / M), so the chunk epilogue in the main
    // loop issues no global load (whose wait would also wait for the code loads in flight)
    float *s_sa = (float *)(smem + ((fp4_tables_bytes<JPF, LUTSRC>(P) + 15) & ~15));
    float *s_sb = s_sa + nchunks * TR;
    fp4_load_tables<JPF, LUTSRC, NT>(P, sA, sB);
    if (SLDS) {
        for (int e = tid; e < nchunks * TR; e += NT) {
            const int k = e / TR, r = e - k * TR;
            s_sa[e] = tr0 + r < P.N ? P.epi.sa[(int64_t)k * P.epi.sa_chunk_stride + tr0 + r] : 0.f;
        }
        for (int e = tid; e < nchunks * TC; e += NT) {
            const int k = e / TC, c = e - k * TC;
            s_sb[e] = tc0 + c < P.M ? P.epi.sb[(int64_t)k * P.epi.sb_chunk_stride + tc0 + c] : 0.f;
        }
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, li = lane & 31;
    const int wa = wave % WA, wb = wave / WA;
    const int a0 = tr0 + wa * (BA * 32);
    const int b0 = tc0 + wb * (BB * 32);

    const uint8_t *abase = P.ca + batch * P.bsa + (int64_t)a0 * P.lda;
    const uint8_t *bbase = P.cb + batch * P.bsb + (int64_t)b0 * P.ldb;

    v16f acc[BA][BB];
    float yac[BA][BB][16];
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int c = 0; c < BB; ++c) {
            acc[i][c] = (v16f){0.0f};
#pragma unroll
            for (int r = 0; r < 16; ++r) yac[i][c][r] = 0.0f;
        }
    const int chunk = P.chunk;
    int kchunk = 0;

    // fp32 sum over inner-dimension chunks, in chunk order (sc/kernels.py:1333-1381):
    // y += fl(fl(I_chunk * c) * fl(sa_chunk * sb_chunk)) after the chunk's last d
    auto after = [&](int dfirst, int dl) __attribute__((always_inline)) {
        if (dfirst >= D) return;
        const int dlast = dl < D ? dl : D - 1;
        if (!(((dlast + 1) % chunk == 0) || (dlast + 1 >= D))) return;
        const float cc = P.epi.c;
        const float *sa = P.epi.sa + (int64_t)kchunk * P.epi.sa_chunk_stride;
        const float *sb = P.epi.sb + (int64_t)kchunk * P.epi.sb_chunk_stride;
        const int lsa0 = kchunk * TR - tr0;                  // s_sa[lsa0 + n]: row n
        const int lsb0 = kchunk * TC - tc0;                  // s_sb[lsb0 + m]: column m
#pragma unroll
        for (int c = 0; c < BB; ++c) {
            const int m = b0 + 32 * c + li;
            const float sbm = SLDS ? s_sb[lsb0 + m] : (m < P.M ? sb[m] : 0.0f);
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = a0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    const float san = SLDS ? s_sa[lsa0 + n] : (n < P.N ? sa[n] : 0.0f);
                    const float raw = __fmul_rn(acc[i][c][r], cc);
                    const float term = __fmul_rn(raw, __fmul_rn(san, sbm));
                    yac[i][c][r] = __fadd_rn(yac[i][c][r], term);
                    acc[i][c][r] = 0.0f;
                }
        }
        ++kchunk;
    };
    fp4_accumulate<JPF, BA, BB, LUTSRC, false>(P, sA, sB, abase, bbase, li, 0, ngroups, h, acc,
                                               after);

    // two store loops so that the common one (no row map) issues no loads between stores
    float *__restrict__ ybat = P.y + batch * P.bsy;
    if (P.row_map == nullptr) {
#pragma unroll
        for (int c = 0; c < BB; ++c) {
            const int m = b0 + 32 * c + li;
            if (m >= P.M) continue;
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = a0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (n < P.N) ybat[(int64_t)n * P.ldy + m] = yac[i][c][r];
                }
        }
    } else {
#pragma unroll
        for (int c = 0; c < BB; ++c) {
            const int m = b0 + 32 * c + li;
            if (m >= P.M) continue;
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = a0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (n < P.N) ybat[P.row_map[n] * P.ldy + m] = yac[i][c][r];
                }
        }
    }
}

// Largest LDS request of one workgroup (gfx950: 160 KiB per CU).
constexpr int kFp4MaxLds = 160 * 1024;

template <class K>
static int fp4_set_lds(K kern, size_t lds, size_t static_lds) {
    if (lds + static_lds <= 64 * 1024) return SCMP_OK;
    if (lds + static_lds > (size_t)kFp4MaxLds) {
        set_error("scmp_sc_gemm(mfma fp4): %zu + %zu bytes of LDS exceed %d", lds, static_lds,
                  kFp4MaxLds);
        return SCMP_E_ARG;
    }
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
        set_error("scmp_sc_gemm(mfma fp4): %zu bytes of LDS refused: %s", lds,
                  hipGetErrorString(e));
        return SCMP_E_LAUNCH;
    }
    return SCMP_OK;
}

// dynamic LDS of the stream tables (the thermometer table, Fp4Geom<JPF>::TAB bytes, is static)
template <int JPF, int LUTSRC>
static size_t fp4_tables_bytes_host(const GemmP &P) {
    using G = Fp4Geom<JPF>;
    return (size_t)G::TAB * (LUTSRC == LUT_LDS || LUTSRC == LUT_RUNS ? 1
                             : LUTSRC == LUT_LDS_CLASSES                ? P.nclass
                                                                        : 0);
}

// Non-chunked, tile shape SHAPE (waves of 4 x 4 blocks of 32 x 32, narrow: 2 x 2);
// epilogue fused; P.nwg persistent workgroups
// (P.ntiles when no split workspace was given: one tile each, no partial sums).
template <int JPF, int LUTSRC, int SHAPE = TILE_SQUARE>
static int launch_fp4_main(const GemmP &P0, int64_t batch, hipStream_t stream) {
    constexpr bool NARROW = SHAPE == TILE_NARROW, T224 = SHAPE == TILE_224;
    constexpr int BA = NARROW || T224 ? 2 : 4, BB = NARROW ? 2 : T224 ? 7 : 4,
                  WA = NARROW || T224 ? 4 : SHAPE == TILE_WIDE ? 1 : 2,
                  WB = NARROW || T224 ? 1 : SHAPE == TILE_WIDE ? 4 : 2;
    GemmP P = P0;
    // MFMA / LDS-read interleaving pinned for JPF = 16, 64 and >= 128; for JPF = 32 the
    // compiler's own schedule measured 9.5% faster
    constexpr bool SCHED = JPF != 32;
    auto kern = sc_gemm_fp4_kernel<JPF, BA, BB, WA, WB, LUTSRC, SCHED>;
    const size_t lds = ((fp4_tables_bytes_host<JPF, LUTSRC>(P) + 15) & ~(size_t)15) +
                       (size_t)(kFactorFloats + WA * WB * kStageFloats) * sizeof(float);
    int rc = fp4_set_lds(kern, lds, Fp4Geom<JPF>::TAB);
    if (rc != SCMP_OK) return rc;
    kern<<<dim3((unsigned)P.nwg), 64 * WA * WB, lds, stream>>>(P);
    SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma fp4)");
    if (P.deferred && P.nwg > 1) {
        const dim3 grid((unsigned)P.ntiles, (unsigned)(WA * WB * BA * BB));
        switch (P.epi.kind) {
        case SCMP_EPI_INT:
            sc_gemm_fp4_fixup_kernel<SCMP_EPI_INT, BA, BB, WA, WB><<<grid, 256, 0, stream>>>(P);
            break;
        case SCMP_EPI_ROWCOL:
            sc_gemm_fp4_fixup_kernel<SCMP_EPI_ROWCOL, BA, BB, WA, WB><<<grid, 256, 0, stream>>>(P);
            break;
        case SCMP_EPI_SCALAR:
            sc_gemm_fp4_fixup_kernel<SCMP_EPI_SCALAR, BA, BB, WA, WB><<<grid, 256, 0, stream>>>(P);
            break;
        case SCMP_EPI_HEAD:
            sc_gemm_fp4_fixup_kernel<SCMP_EPI_HEAD, BA, BB, WA, WB><<<grid, 256, 0, stream>>>(P);
            break;
        case SCMP_EPI_ZP_ROWCOL:
            sc_gemm_fp4_fixup_kernel<SCMP_EPI_ZP_ROWCOL, BA, BB, WA, WB><<<grid, 256, 0, stream>>>(P);
            break;
        default:
            sc_gemm_fp4_fixup_kernel<SCMP_EPI_ZP_SCALAR, BA, BB, WA, WB><<<grid, 256, 0, stream>>>(P);
            break;
        }
        SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma fp4 fixup)");
    }
    return SCMP_OK;
}

// LDS bytes of the chunked kernel's stream tables and per-chunk scales for TR-row tiles
template <int JPF, int LUTSRC>
static size_t chunked_lds(const GemmP &P, int TR, size_t *tabs_out) {
    const size_t tabs = (fp4_tables_bytes_host<JPF, LUTSRC>(P) + 15) & ~(size_t)15;
    if (tabs_out) *tabs_out = tabs;
    return tabs + (size_t)cdiv(P.D, P.chunk) * (TR + 128) * sizeof(float);
}

// 256-row tiles only with every chunk scale in LDS: without, or with 32-interval per-d class
// tables, the 128 x 64 wave tile spills its registers
template <int JPF, int LUTSRC>
static bool chunked_tall_ok(const GemmP &P) {
    if constexpr (JPF == 32 && LUTSRC != LUT_LDS) return false;
    return Fp4Geom<JPF>::TAB + chunked_lds<JPF, LUTSRC>(P, 256, nullptr) <= (size_t)kFp4MaxLds;
}

// Chunked launch of rows [P.row0, P.N) in TR x 128 tiles (TR = 64 BA), BA x 2 blocks of
// 32 x 32 per wave (fp32 chunk sums in registers), one workgroup per tile.
template <int JPF, int LUTSRC, int BA>
static int launch_fp4_chunked_rows(const GemmP &P0, int64_t batch, hipStream_t stream) {
    constexpr int BB = 2, WA = 2, WB = 2;
    if constexpr (BA == 4 && JPF == 32 && LUTSRC != LUT_LDS) {
        set_error("scmp_sc_gemm(mfma fp4, chunked): no 256-row tiles for these tables");
        return SCMP_E_ARG;
    } else {
        GemmP P = P0;
        P.tilesA = (int)cdiv(P.N - P.row0, WA * BA * 32);
        const int64_t tilesB = cdiv(P.M, WB * BB * 32);
        size_t tabs = 0;
        const size_t with_scales = chunked_lds<JPF, LUTSRC>(P, WA * BA * 32, &tabs);
        const bool slds = Fp4Geom<JPF>::TAB + with_scales <= (size_t)kFp4MaxLds;
        auto kern = sc_gemm_fp4_chunked_kernel<JPF, BA, BB, WA, WB, LUTSRC, true>;
        if constexpr (BA == 4) {
            if (!chunked_tall_ok<JPF, LUTSRC>(P)) {
                set_error("scmp_sc_gemm(mfma fp4, chunked): 256-row tiles planned without room");
                return SCMP_E_ARG;
            }
        } else {
            if (!slds) kern = sc_gemm_fp4_chunked_kernel<JPF, BA, BB, WA, WB, LUTSRC, false>;
        }
        const size_t lds = slds ? with_scales : tabs;
        int rc = fp4_set_lds(kern, lds, Fp4Geom<JPF>::TAB);
        if (rc != SCMP_OK) return rc;
        kern<<<dim3((unsigned)(P.tilesA * tilesB), 1, (unsigned)batch), 64 * WA * WB, lds,
               stream>>>(P);
        SCMP_LAUNCH_CHECK("scmp_sc_gemm(mfma fp4, chunked)");
        return SCMP_OK;
    }
}

// Row plan of the chunked kernel: rows [0, rows_main) in main_rows x 128 tiles, the rest in
// tail_rows x 128 tiles (a second launch; tail_rows 0: none).
struct ChunkPlan {
    int main_rows, tail_rows;
    int64_t rows_main;
};

// Chunked: one workgroup per tile and compute unit. The inner dimension cannot be split (the
// fp32 chunk sums have a fixed order), so the tiles run in rounds of one per compute unit and
// the tile height sets both the rounds and the work of each. The kernel is bound by LDS
// reads of the tables: a 128 x 128 tile (64 x 64 per wave) reads one 16-byte fragment per
// lane and MFMA, a 256 x 128 tile (128 x 64 per wave: twice the MFMAs, its fp32 chunk sums
// and accumulators fill the registers) 0.75, a 64 x 128 tile (32 x 64 per wave: half the
// MFMAs) 1.5. Measured time of a round in tenths of a 128 x 128 round (cfg3's tiles): 256
// rows 16, 128 rows 10, 64 rows 6. The plan is the cheapest of: all
// rows in 128-row tiles; full rounds of 256-row (when `tall`) or 128-row tiles with the
// remaining rows in 64- or 128-row tiles.
static ChunkPlan chunk_plan(int64_t N, int64_t per_row_tile, int64_t ncu, bool tall) {
    auto rounds = [&](int64_t rows, int tr) { return cdiv(cdiv(rows, tr) * per_row_tile, ncu); };
    auto cost_of = [](int tr) { return tr == 256 ? 16 : tr == 128 ? 10 : 6; };
    ChunkPlan best{128, 0, N};
    int64_t best_cost = 10 * rounds(N, 128);
    for (int mr : {256, 128}) {
        if (mr == 256 && !tall) continue;
        const int64_t per_round = ncu / per_row_tile;         // row tiles one round holds
        for (int64_t k = 1; per_round > 0 && k * per_round * mr < N; ++k) {
            const int64_t rows_main = k * per_round * mr;
            for (int tr : {64, 128}) {
                const int64_t c = k * cost_of(mr) + cost_of(tr) * rounds(N - rows_main, tr);
                if (c < best_cost) {
                    best_cost = c;
                    best = ChunkPlan{mr, tr, rows_main};
                }
            }
        }
    }
    return best;
}

template <int JPF, int LUTSRC>
static int launch_chunked_part(const GemmP &P, int tile_rows, int64_t batch, hipStream_t stream) {
    if (tile_rows == 256) return launch_fp4_chunked_rows<JPF, LUTSRC, 4>(P, batch, stream);
    if (tile_rows == 64) return launch_fp4_chunked_rows<JPF, LUTSRC, 1>(P, batch, stream);
    return launch_fp4_chunked_rows<JPF, LUTSRC, 2>(P, batch, stream);
}

template <int JPF, int LUTSRC>
static int launch_fp4_chunked(const GemmP &P, int64_t batch, hipStream_t stream) {
    const ChunkPlan plan =
        chunk_plan(P.N, cdiv(P.M, 128) * batch, P.nwg, chunked_tall_ok<JPF, LUTSRC>(P));
    if (plan.tail_rows == 0) return launch_chunked_part<JPF, LUTSRC>(P, plan.main_rows, batch, stream);
    GemmP Pm = P;
    Pm.N = (int)plan.rows_main;                            // rows [0, rows_main)
    int rc = launch_chunked_part<JPF, LUTSRC>(Pm, plan.main_rows, batch, stream);
    if (rc != SCMP_OK) return rc;
    GemmP Pt = P;
    Pt.row0 = (int)plan.rows_main;                         // rows [rows_main, N)
    return launch_chunked_part<JPF, LUTSRC>(Pt, plan.tail_rows, batch, stream);
}

// Stream tables: one shared table in LDS; every class table in LDS when they fit
// (leaving room for the epilogue staging); otherwise per-class rows from global memory.
template <int JPF>
int gemm_fp4_launch_jpf(const GemmP &P, int64_t batch, bool chunked, hipStream_t s) {
    using G = Fp4Geom<JPF>;
    if constexpr (JPF == 16) {
        if (chunked) {                           // the chunk_d kernel takes such tables as 32
            set_error("scmp_sc_gemm(fp4): chunked launch with JPF=16");
            return SCMP_E_ARG;
        }
    }
    // the non-chunked kernel in the planned tile shape (narrow: single table only)
    auto main_kernel = [&](auto src) {
        constexpr int SRC = decltype(src)::value;
        return P.tile_cols == 512 ? launch_fp4_main<JPF, SRC, TILE_WIDE>(P, batch, s)
                                  : launch_fp4_main<JPF, SRC>(P, batch, s);
    };
    using Lds = std::integral_constant<int, LUT_LDS>;
    using Classes = std::integral_constant<int, LUT_LDS_CLASSES>;
    using Global = std::integral_constant<int, LUT_GLOBAL>;
    using Runs = std::integral_constant<int, LUT_RUNS>;
    const int64_t stage = (kFactorFloats + 4 * kStageFloats) * (int64_t)sizeof(float);
    if (P.group_class != nullptr) {
        if (chunked || P.d_class != nullptr || P.nclass <= 0) {
            set_error("scmp_sc_gemm(fp4): group_class needs a non-chunked launch, no d_class "
                      "and nclass > 0");
            return SCMP_E_ARG;
        }
        return main_kernel(Runs{});
    }
    if (P.d_class == nullptr) {
        if constexpr (JPF != 16)
            if (chunked) return launch_fp4_chunked<JPF, LUT_LDS>(P, batch, s);
        if (P.tile_cols == 224) return launch_fp4_main<JPF, LUT_LDS, TILE_224>(P, batch, s);
        return P.tile_cols == 64 ? launch_fp4_main<JPF, LUT_LDS, TILE_NARROW>(P, batch, s)
                                 : main_kernel(Lds{});
    }
    const bool fits = P.nclass > 0 && (int64_t)G::TAB * (1 + P.nclass) + stage <= kFp4MaxLds;
    if constexpr (JPF != 16) {
        if (chunked)
            return fits ? launch_fp4_chunked<JPF, LUT_LDS_CLASSES>(P, batch, s)
                        : launch_fp4_chunked<JPF, LUT_GLOBAL>(P, batch, s);
    }
    return fits ? main_kernel(Classes{}) : main_kernel(Global{});
}

}  // namespace scmp
