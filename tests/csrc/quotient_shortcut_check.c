// CPU check of the quantizers' quotient shortcut (scmp_kernels_amd/csrc/quant.hip,
// rne_quotient and the codes-only chunk path): rne(fl(x / s)) and rne(fl(fl(x / s) + zp))
// equal the result of y = fl(x * fl(1 / s)) whenever |y| < 1024 and y (or fl(y + zp)) is
// farther than 2^-11 from every half-integer; other inputs take the exact division.
// Samples: in-range values, values within 1e-4 of half-integers, values far beyond the
// clamp, and tiny values, for group scales over 60 binades and Q = 127 / 255.
// Built with -ffp-contract=off: every operation rounds once, as on the GPU.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
static uint64_t st = 88172645463325252ull;
static uint64_t xr(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static float uf(void) { return (float)((xr() >> 11) * (1.0 / 9007199254740992.0)); }
static float fast_sym(float x, float s, float inv) {
    volatile float y = x * inv;
    float k = rintf(y);
    float f = fabsf(y - k);
    if (fabsf(y) < 1024.0f && f < 0.5f - 4.8828125e-4f) return k;
    volatile float t = x / s;
    return rintf(t);
}
static float fast_asym(float x, float s, float inv, float zp) {
    volatile float y = x * inv;
    if (fabsf(y) < 1024.0f) {
        volatile float u = y + zp;
        float k = rintf(u);
        float f = fabsf(u - k);
        if (f < 0.5f - 4.8828125e-4f) return k;
    }
    volatile float t = x / s;
    volatile float t2 = t + zp;
    return rintf(t2);
}
int main(int argc, char **argv) {
    long n = argc > 1 ? atol(argv[1]) : 100000000L;
    long bad = 0, slow = 0;
    for (long i = 0; i < n; ++i) {
        float A = ldexpf(uf() + 0.5f, (int)(xr() % 60) - 40);     // group absmax
        if (A < 1e-5f) A = 1e-5f;
        float Q = (xr() & 1) ? 127.0f : 255.0f;
        volatile float s = A / Q;
        volatile float inv = 1.0f / s;
        float x;
        int mode = xr() % 4;
        if (mode == 0) x = (uf() * 2 - 1) * A;                        // in range
        else if (mode == 1) {                                          // near half-integers
            float k = floorf(uf() * Q) + 0.5f;
            x = (k + (uf() - 0.5f) * 1e-4f) * s * ((xr() & 1) ? 1 : -1);
        } else if (mode == 2) x = (uf() * 2 - 1) * A * 2000.0f;      // beyond the clamp
        else x = ldexpf(uf(), -(int)(xr() % 140));                     // tiny
        float r1 = rintf((volatile float)(x / s));
        float r2 = fast_sym(x, s, inv);
        if (r1 != r2 || signbit(r1) != signbit(r2)) { if (bad++ < 10) printf("sym x=%a s=%a %g %g\n", x, s, r1, r2); }
        float zp = floorf(uf() * (Q + 1));
        volatile float t = x / s; volatile float t2 = t + zp;
        float r3 = rintf(t2);
        float r4 = fast_asym(x, s, inv, zp);
        if (r3 != r4 || signbit(r3) != signbit(r4)) { if (bad++ < 10) printf("asym x=%a s=%a zp=%g %g %g\n", x, s, zp, r3, r4); }
        volatile float y = x * inv;
        if (!(fabsf(y) < 1024.0f) || fabsf(y - rintf(y)) >= 0.5f - 4.8828125e-4f) slow++;
    }
    printf("n=%ld mismatches=%ld slow-path fraction=%.3g\n", n, bad, (double)slow / n);
    return bad != 0;
}
