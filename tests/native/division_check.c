/*
 * Exhaustive CPU check of the division method the HIP quantizers use.
 *
 * The kernels replace the per-element IEEE binary32 quotient x / s by
 *     r  = RN(1 / s)            (one correctly rounded division per row)
 *     q0 = RN(x * r)
 *     e  = -fma(q0, s, -x)      (exact remainder x - q0*s)
 *     q  = RN(q0 + e * r)       (one fma)
 * The remainder is spelled -fma(q0, s, -x) rather than fma(-q0, s, x) so that
 * x = -0 gives e = -0 and q = -0: the other spelling returns +0 and loses the
 * sign that torch's cast keeps (code 0x80).
 * Markstein's theorem says q == RN(x / s) when r is the correctly rounded
 * reciprocal and no overflow/underflow intervenes.  This program checks the
 * claim for EVERY input the quantizers can see: s ranges over the scales
 * max(RN(a / 448), 1e-12) for every finite bf16 row maximum a (and, for the
 * weight path, over bf16(s) too), and x over every bf16 value with |x| <= a.
 * The comparison is on what the quantizers store: the e4m3 code of the
 * quotient (activation path) and the e4m3 code of its bf16 rounding (weight
 * path).  Raw binary32 quotients differ only where x is a bf16 subnormal and
 * the remainder underflows; there the quotient is below 2^-26 and encodes to
 * a signed zero either way, which this program confirms.
 * For the weight path the kernels go further: there x and bf16(s) are both
 * bf16, and the single product RN(x * r) rounds to the same bf16 value as the
 * IEEE quotient for every pair (an 8-bit by 8-bit quotient never lies within
 * the product's error of a bf16 rounding midpoint); this is checked too.
 * Returns nonzero on any mismatch and prints a summary.
 *
 * Build: gcc -O2 -ffp-contract=off -fopenmp division_check.c ../../oracle/fp8_oracle.c -lm -lpthread
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float b2f(uint16_t h) { uint32_t u = (uint32_t)h << 16; float f; memcpy(&f, &u, 4); return f; }
static uint16_t f2b(float f) { uint32_t u; memcpy(&u, &f, 4); u += 0x7fffu + ((u >> 16) & 1u); return (uint16_t)(u >> 16); }

/* fp32 -> e4m3 (RNE, |x| > 464 -> NaN, sign kept): the oracle's encoder. */
uint8_t oracle_e4m3_from_f32(float f);

static long raw_mismatch_total = 0, raw_mismatch_big = 0, mul_mismatch_total = 0;

static long check_scale(float s, uint16_t amax_bits, int weight_path)
{
    long bad = 0, raw = 0, raw_big = 0, bad_mul = 0;
    float r = 1.0f / s;
    for (uint32_t h = 0; h <= amax_bits; ++h) {
        for (int sg = 0; sg < 2; ++sg) {
            float x = b2f((uint16_t)(h | (sg ? 0x8000u : 0u)));
            float want = x / s;
            float q0 = x * r;
            float e = -fmaf(q0, s, -x);
            float q = fmaf(e, r, q0);
            uint32_t a, b;
            memcpy(&a, &want, 4);
            memcpy(&b, &q, 4);
            if (a != b) {
                ++raw;
                if (fabsf(want) >= 0x1p-26f) ++raw_big;
            }
            if (weight_path) {
                /* the weight path stores bf16(quotient) and both operands are bf16:
                 * there the kernels use the single multiply x * r, whose bf16
                 * rounding must equal that of the IEEE quotient, bit for bit */
                const uint16_t wb = f2b(want), mb = f2b(x * r);
                if (wb != mb) ++bad_mul;
                want = b2f(wb);
                q = b2f(f2b(q));
            }
            if (oracle_e4m3_from_f32(want) != oracle_e4m3_from_f32(q)) ++bad;
        }
    }
#pragma omp atomic
    raw_mismatch_total += raw;
#pragma omp atomic
    raw_mismatch_big += raw_big;
#pragma omp atomic
    mul_mismatch_total += bad_mul;
    return bad;
}

int main(void)
{
    long bad_act = 0, bad_w = 0;
    /* every finite positive bf16 row maximum (and zero) */
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad_act, bad_w)
    for (int32_t ab = 0; ab < 0x7f80; ++ab) {
        float a = b2f((uint16_t)ab);
        float s = a / 448.0f;
        if (s < 1e-12f) s = 1e-12f;
        bad_act += check_scale(s, (uint16_t)ab, 0);
        bad_w += check_scale(b2f(f2b(s)), (uint16_t)ab, 1);
    }
    printf("code mismatches: activation %ld, weight %ld\n", bad_act, bad_w);
    printf("raw binary32 quotient mismatches: %ld (of which |q| >= 2^-26: %ld)\n",
           raw_mismatch_total, raw_mismatch_big);
    printf("weight path, single multiply: bf16 mismatches %ld\n", mul_mismatch_total);
    return (bad_act + bad_w + raw_mismatch_big + mul_mismatch_total) != 0;
}
