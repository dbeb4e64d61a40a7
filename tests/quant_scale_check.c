/* Checks the quantiser's divide-free scale, fma(x, Ch, RN(x * Cl)) with
 * Ch = RN(1/127) and Cl = RN(1/127 - Ch), against the IEEE quotient x / 127
 * (the oracle's scale) bit for bit, for every float x >= 2^-112:
 * - every x in [2^-112, 2^-90): there x * Cl or the quotient is subnormal,
 *   so the result depends on the exponent;
 * - every significand in one binade, [1, 2): for x in [2^-90, 2^128) every
 *   intermediate and the result are normal, so both sides scale exactly by
 *   powers of two and one binade decides all of them;
 * - the binade boundaries' neighbours and +Inf, directly.
 * Also reports that x just below 2^-112 does differ, so the device keeps the
 * divide there.  Exit status 0 when every check holds.
 * Built with -ffp-contract=off so that x * Cl is rounded on its own (OpenMP
 * optional). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static const float kCh = 0x1.020408p-7f;
#ifdef PLANT_NO_LOW_PART /* a planted mistake: the low part dropped */
static const float kCl = 0.0f;
#else
static const float kCl = 0x1.020408p-35f;
#endif

static float scale_fast(float x) {
    volatile float lo = x * kCl;
    return fmaf(x, kCh, lo);
}

static uint32_t bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

static float from_bits(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

static int same(float x) {
    volatile float d = x / 127.0f;
    return bits(scale_fast(x)) == bits(d);
}

int main(void) {
    if ((double)kCh != (double)(float)(1.0 / 127.0)) {
        printf("Ch differs from RN(1/127)\n");
        return 1;
    }
    unsigned long long bad = 0, checked = 0;
    const long long lo1 = bits(0x1p-112f), hi1 = bits(0x1p-90f), lo2 = bits(1.0f), hi2 = bits(2.0f);
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = lo1; u < hi1; u++) bad += !same(from_bits((uint32_t)u));
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = lo2; u < hi2; u++) bad += !same(from_bits((uint32_t)u));
    checked += (unsigned long long)(hi1 - lo1 + hi2 - lo2);
    for (int e = -90; e < 128; e++) {
        const float b = ldexpf(1.0f, e);
        const float probe[3] = {nextafterf(b, 0.0f), b, nextafterf(b, INFINITY)};
        for (int i = 0; i < 3; i++, checked++) bad += !same(probe[i]);
    }
    bad += !same(INFINITY);
    checked++;
    unsigned long long below = 0;
    for (uint32_t u = bits(0x1p-113f); u < bits(0x1p-112f); u++) below += !same(from_bits(u));
    printf("checked %llu mismatches %llu below-2^-112 mismatches %llu\n", checked, bad, below);
    return bad != 0 || below == 0;
}
