/* Host check of the division identity the apply kernel relies on
 * (gefenx_device.h div_by_block): with y = RN(1/b), q0 = RN(u*y),
 * r = fma(-q0, b, u), RN(fma(r, y, q0)) == RN(u/b) whenever |u| and |q0| are
 * at least 2^-100 and b lies in [2^-125, 2^125].  Exhaustive over a band of
 * divisor significands plus random pairs with |u| <= b (the kernel's domain:
 * b is the block max of |u|).  Prints the number of mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static float div_by_block(float u, float b, float y) {
    if (y != 0.0f && fabsf(u) >= 0x1p-100f) {
        float q0 = u * y;
        if (fabsf(q0) >= 0x1p-100f) {
            float r = fmaf(-q0, b, u);
            return fmaf(r, y, q0);
        }
    }
    return u / b;
}

/* gefenx_device.h div_by_const: the same step for any quotient size, with
 * the range guards that keep it away from under- and overflow. */
static float div_by_const(float u, float d, float y) {
    float q0 = u * y;
    float aq = fabsf(q0);
    if (y != 0.0f && fabsf(u) >= 0x1p-100f && fabsf(u) <= 0x1p100f && aq >= 0x1p-100f && aq <= 0x1p100f) {
        float r = fmaf(-q0, d, u);
        return fmaf(r, y, q0);
    }
    return u == 0.0f && y != 0.0f ? q0 : u / d;
}

static float block_recip(float b) {
    if (!(b >= 0x1p-125f) || !(b <= 0x1p125f)) return 0.0f;
    return 1.0f / b;
}

static uint64_t s = 0x9E3779B97F4A7C15ULL;
static uint64_t next(void) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

int main(int argc, char** argv) {
    long n = argc > 1 ? atol(argv[1]) : 20000000L;
    long bad = 0, checked = 0;
    for (long i = 0; i < n; ++i) {
        uint64_t r = next();
        /* divisor: random significand, exponent in [-40, 10] */
        int e = (int)(r % 51) - 40;
        float b = ldexpf(1.0f + (float)((r >> 8) & 0x7fffff) / 8388608.0f, e);
        float y = block_recip(b);
        /* numerator: |u| <= b, spread over many binades below b */
        uint64_t r2 = next();
        int de = (int)(r2 % 40);
        float u = ldexpf(1.0f + (float)((r2 >> 8) & 0x7fffff) / 8388608.0f, e - de);
        if (u > b) u = b;
        if (r2 & (1ULL << 60)) u = -u;
        float got = div_by_block(u, b, y);
        float want = u / b;
        ++checked;
        if (memcmp(&got, &want, 4) != 0) {
            if (bad < 10) fprintf(stderr, "mismatch u=%a b=%a got=%a want=%a\n", u, b, got, want);
            ++bad;
        }
    }
    /* every significand of b in a window, u = largest values below b and the
     * edges of the binade */
    for (uint32_t m = 0; m < (1u << 16); ++m) {
        float b = fbits(0x3f800000u | (m << 7) | (m & 0x7f));
        float y = block_recip(b);
        float us[6] = {b, -b, nextafterf(b, 0.0f), 1.0f, 0.5f * b, fbits(0x3f800001u)};
        for (int k = 0; k < 6; ++k) {
            float u = us[k];
            if (fabsf(u) > b) continue;
            float got = div_by_block(u, b, y), want = u / b;
            ++checked;
            if (memcmp(&got, &want, 4) != 0) {
                if (bad < 10) fprintf(stderr, "mismatch u=%a b=%a got=%a want=%a\n", u, b, got, want);
                ++bad;
            }
        }
    }
    /* div_by_const: random numerators and divisors over wide exponent ranges
     * (quotients far above and below 1, zeros, the guard edges) */
    for (long i = 0; i < n; ++i) {
        uint64_t r = next(), r2 = next();
        int ed = (int)(r % 241) - 120;
        float d = ldexpf(1.0f + (float)((r >> 8) & 0x7fffff) / 8388608.0f, ed);
        int eu = (int)(r2 % 253) - 126;
        float u = ldexpf(1.0f + (float)((r2 >> 8) & 0x7fffff) / 8388608.0f, eu);
        if ((r2 >> 40) % 97 == 0) u = 0.0f;
        if (r2 & (1ULL << 61)) u = -u;
        float y = block_recip(d);
        float got = div_by_const(u, d, y), want = u / d;
        ++checked;
        if (memcmp(&got, &want, 4) != 0 && !(got != got && want != want)) {
            if (bad < 10) fprintf(stderr, "div_by_const mismatch u=%a d=%a got=%a want=%a\n", u, d, got, want);
            ++bad;
        }
    }
    printf("%ld %ld\n", bad, checked);
    return bad != 0;
}
