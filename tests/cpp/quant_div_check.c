/* Exhaustive check of the quotient the GPU quantiser's fast path uses
 * (infer_amd/csrc/iq_quant.hip, qdiv_fast): for bf16 w and a bf16 scale s,
 * t = w * r, q = fma(fma(-t, s, w), r, t) with r within one ulp of 1 / s
 * must equal the correctly rounded fp32 quotient w / s, the value the
 * reference rounds with lrint (src/quant.cpp:56-57, 70-76).
 * Every pair of bf16 significands, both signs, every ratio exponent from
 * 2^-30 to 2^9 (|w / s| <= 2^10 covers the int8 and int4 code ranges), r
 * the correctly rounded reciprocal and its two neighbours, at scale
 * exponents near the fast path's lower limit (2^-64), near 1 and near the
 * top of the fp32 range.  Prints the number of pairs and of mismatches.
 */
#include <math.h>
#include <stdio.h>

static int check_scale_exponent(int es, long* pairs) {
    long bad = 0;
    for (int S = 0; S < 128; S++) {
        const float s = ldexpf(1.0f + S / 128.0f, es);
        const float r0 = 1.0f / s;
        for (int dr = -1; dr <= 1; dr++) {
            const float r = dr == 0 ? r0 : nextafterf(r0, dr < 0 ? 0.0f : INFINITY);
            for (int ew = es - 30; ew <= es + 9; ew++) {
                for (int W = 0; W < 128; W++) {
                    for (int sg = 0; sg < 2; sg++) {
                        float w = ldexpf(1.0f + W / 128.0f, ew);
                        if (sg) w = -w;
                        const float t = w * r;
                        const float q = fmaf(fmaf(-t, s, w), r, t);
                        *pairs += 1;
                        if (q != w / s) bad++;
                    }
                }
            }
        }
    }
    return (int)(bad > 0);
}

int main(void) {
    long pairs = 0;
    int failed = 0;
    for (int es = -64; es <= -56; es++) failed += check_scale_exponent(es, &pairs);
    for (int es = -4; es <= 4; es++) failed += check_scale_exponent(es, &pairs);
    for (int es = 110; es <= 117; es++) failed += check_scale_exponent(es, &pairs);
    printf("pairs %ld failed_exponents %d\n", pairs, failed);
    return failed ? 1 : 0;
}
