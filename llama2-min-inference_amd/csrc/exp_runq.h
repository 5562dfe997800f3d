// exp_runq.h - single-precision exp with the exact results of the host C
// library the reference runner links (glibc expf on x86-64), usable on the
// host and on the GPU.
//
// The reference evaluates expf in its softmax (runq.c:314) and SwiGLU
// (runq.c:407).  A quantized decoder amplifies a 1-ulp difference there:
// an activation sitting on a rounding boundary of x/s moves by one step and
// the greedy ids drift apart within a few dozen tokens.  The GPU therefore
// uses this restatement instead of its own expf.
//
// Method (published: the single-precision exp of Arm's optimized-routines
// library, Szabolcs Nagy 2017, the implementation glibc >= 2.28 ships):
// in double precision,
//     z  = x * 32/ln2,   k = nearest integer to z,   r = z - k
//     2^(k/32) from a 32-entry table of 2^(i/32) with k>>5 added to the
//     exponent field,
//     2^(r/32) ~ 1 + c2 r + c1 r^2 + c0 r^3   (coefficients scaled by 32^-n)
//     result = (float)(2^(k/32) * poly(r)).
// The table is 2^(i/32) correctly rounded to double (generated with Python
// decimal at 60 digits); r is formed with one fused multiply-add, the form
// the FMA build of the host library uses.  The restatement equals the host
// expf on every float in (-103.97, 88.72) - verified exhaustively by the
// test suite - and reproduces its overflow / underflow / NaN boundaries.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define L2Q_HD __host__ __device__
#else
#define L2Q_HD
#endif

namespace l2q {

#if defined(__HIPCC__)
__device__ __constant__
#endif
static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

L2Q_HD inline uint64_t bits_of(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}
L2Q_HD inline double double_of(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}
L2Q_HD inline uint32_t bits_of(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// tab: kExp2Tab or a copy of it (a kernel may keep one in LDS so that the
// lookup is not a global load queued behind its weight stream).
L2Q_HD inline float exp_runq_t(float x, const uint64_t* tab) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    const double kShift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const uint32_t top = (bits_of(x) >> 20) & 0x7ff;
    if (top >= 0x42b) {                              // |x| >= 88, inf or nan
        if (bits_of(x) == 0xff800000u) return 0.0f;  // -inf
        if (top >= 0x7f8) return x + x;             // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = bits_of(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = double_of(t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

L2Q_HD inline float exp_runq(float x) { return exp_runq_t(x, kExp2Tab); }

}  // namespace l2q
