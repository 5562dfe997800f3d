// expcheck.cpp - host build of the device exp (csrc/exp_runq.h) for the
// identity check against the host C library's expf on every input.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "exp_runq.h"

extern "C" float l2q_exp_runq_host(float x) { return l2q::exp_runq(x); }

// Number of float bit patterns in [lo, hi) where exp_runq and expf differ
// (two NaNs count as equal).
extern "C" long long l2q_exp_runq_mismatches(uint64_t lo, uint64_t hi) {
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = (long long)lo; u < (long long)hi; u++) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const float a = l2q::exp_runq(x), r = expf(x);
        uint32_t ua, ur;
        memcpy(&ua, &a, 4);
        memcpy(&ur, &r, 4);
        if (ua != ur && !(isnan(a) && isnan(r))) bad++;
    }
    return bad;
}
