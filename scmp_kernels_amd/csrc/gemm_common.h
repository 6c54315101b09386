// Definitions shared by the SC GEMM kernels (int8 and FP4 MFMA).
#pragma once

#include "common.h"

namespace scmp {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef char v16c __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Launch parameters of the MFMA SC GEMM kernels (passed by value).
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
    int nclass;
};

int run_epilogue(const int32_t *iin, float *y, int64_t N, int64_t M, int64_t batch,
                 int64_t ldy, int64_t bsy, const scmp_epilogue &E, hipStream_t stream);
int gemm_fp4_launch(const GemmP &P, int64_t batch, int JPF, int tile, bool chunked,
                    hipStream_t stream);

}  // namespace scmp
