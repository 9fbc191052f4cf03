/*
 * fp8_oracle.c -- CPU restatement of the reference's fp8 quantized-linear
 * arithmetic, used ONLY as test infrastructure (what results are compared
 * with): tests/, the
 * smoke check in __graft_entry__.py and the cpu_baseline leg of bench.py load
 * it. Nothing in the product path links, loads or calls this file.
 *
 * Every function states the reference file:line it restates (paths relative
 * to the reference checkout).  The arithmetic is written from the
 * definitions, in plain C99, with IEEE binary32 division and round-to-nearest-
 * even, so that it follows torch's CPU eager spelling that the reference's own
 * tests use as the contract (`quantize_rows_reference`, fp8_linear.py:132-135).
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, never -ffast-math:
 * contraction or reassociation would change the binary32 results).
 *
 * How each function is pinned (checked by tests/test_oracle.py):
 *   oracle_e4m3_from_f32   exhaustive over all bf16 patterns and over every
 *                          e4m3 rounding midpoint +-1 ulp against torch's CPU
 *                          cast and against a nearest-value brute force over
 *                          the 256-entry code table; KATs from the probed cast.
 *   oracle_bf16_from_f32   against torch's CPU cast (random and boundary bits).
 *   oracle_quantize_rows   against the torch-eager restatement of
 *                          quantize_rows_reference; invariants (row max maps to
 *                          +-448, scale floor 1e-12, signed zeros).
 *   oracle_quantize_weight against the torch-eager restatement of the rowwise
 *                          branch of Fp8Linear.__init__ (bf16 double rounding).
 *   oracle_lora_merge      against torch fp32 matmul (<= 1 bf16 ulp) and a
 *                          brute-force exact-sum case.
 *   oracle_swiglu_quantize_rows  parity unpinned beyond tolerance: sigmoid is
 *                          transcendental; checked against torch eager within
 *                          one fp8 code.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar helpers                                                            */
/* ------------------------------------------------------------------------ */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* bf16 -> fp32 is exact: the bf16 pattern is the high half of the fp32 one. */
float oracle_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN -> quiet NaN keeping the sign.
 * Follows torch's Tensor.to(torch.bfloat16) on CPU (used by fp8_linear.py:265
 * through scale.to(weight.dtype) and by the bf16 quotient there). */
uint16_t oracle_bf16_from_f32(float f)
{
    uint32_t u = f32_to_bits(f);
    if (isnan(f)) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

/* e4m3 (OCP "fn" variant: no infinities, 0x7f/0xff are NaN, max 448) decode. */
float oracle_e4m3_to_f32(uint8_t c)
{
    int sign = c >> 7, e = (c >> 3) & 0xf, m = c & 7;
    float v;
    if (e == 0xf && m == 7) return sign ? -NAN : NAN;
    if (e == 0) v = ldexpf((float)m, -9);               /* subnormal: m * 2^-9 */
    else v = ldexpf((float)(8 + m), e - 10);             /* (1 + m/8) * 2^(e-7) */
    return sign ? -v : v;
}

/* fp32 -> e4m3 with round to nearest, ties to even, no saturation -- the
 * semantics of torch's `.to(torch.float8_e4m3fn)` that the reference applies
 * after its scaling (fp8_linear.py:135 and :265):
 *   |x| >  464 (the midpoint between 448 and the NaN pattern) -> NaN
 *   |x| == 464                                                -> 448 (even)
 *   NaN / inf                                                 -> NaN
 *   the sign is always kept, also for zero and for underflow to zero.
 * The code is continuous across the subnormal/normal boundary: for the binade
 * [2^E, 2^(E+1)) with E >= -6 the quantum is 2^(E-3); below 2^-6 it is 2^-9.
 * With n = the value in quanta rounded to nearest even, code = (E+6)*8 + n,
 * and n == 16 rolls into the next binade by itself. */
uint8_t oracle_e4m3_from_f32(float f)
{
    uint8_t sign = signbit(f) ? 0x80 : 0x00;
    float a = fabsf(f);
    if (isnan(a) || a > 464.0f) return sign | 0x7f;
    if (a < 0x1p-6f) {
        /* a * 2^9 is exact in binary32 (power-of-two scaling, no underflow
         * below since a >= 2^-149 maps to >= 2^-140). */
        double n = nearbyint((double)a * 512.0);      /* default mode: RNE */
        return sign | (uint8_t)n;                      /* n <= 8 -> code <= 8 */
    }
    int E;
    (void)frexpf(a, &E);                                /* a = m * 2^E, m in [0.5,1) */
    E -= 1;                                             /* a in [2^E, 2^(E+1)) */
    double n = nearbyint(ldexp((double)a, 3 - E));     /* in [8, 16] */
    int code = (E + 6) * 8 + (int)n;
    if (code > 0x7e) code = 0x7e;                       /* only a == 464 reaches 0x7f */
    return sign | (uint8_t)code;
}

/* ------------------------------------------------------------------------ */
/* threading                                                                 */
/* ------------------------------------------------------------------------ */

typedef void (*row_fn)(void *ctx, int64_t r0, int64_t r1);
struct job { row_fn fn; void *ctx; int64_t r0, r1; };
static void *run_job(void *p) { struct job *j = p; j->fn(j->ctx, j->r0, j->r1); return NULL; }

static void parallel_rows(row_fn fn, void *ctx, int64_t rows, int nthreads)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (rows < nthreads) nthreads = rows > 0 ? (int)rows : 1;
    pthread_t th[256];
    struct job jobs[256];
    int64_t per = (rows + nthreads - 1) / nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; ++t) {
        int64_t r0 = t * per, r1 = r0 + per < rows ? r0 + per : rows;
        if (r0 >= r1) break;
        jobs[t] = (struct job){fn, ctx, r0, r1};
        if (nthreads == 1) { run_job(&jobs[t]); continue; }
        pthread_create(&th[t], NULL, run_job, &jobs[t]);
        ++started;
    }
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
}

/* NaN-propagating max, as torch's amax (a NaN anywhere makes the result NaN). */
static inline float nanmax(float a, float b) { return (isnan(a) || a >= b) ? a : b; }
/* torch.clamp_min(scale, 1e-12): NaN stays NaN; the Python float 1e-12 becomes
 * the binary32 value 9.99999996e-13 on a float32 tensor. */
static inline float clamp_floor(float s) { return (s < 1e-12f) ? 1e-12f : s; }

/* ------------------------------------------------------------------------ */
/* per-token activation quantization                                         */
/* ------------------------------------------------------------------------ */

/* Restates quantize_rows_reference (fp8_linear.py:132-135):
 *   scale = (x.float().abs().amax(dim=1, keepdim=True) / 448).clamp_min(1e-12)
 *   y     = (x.float() / scale).to(float8_e4m3fn)
 * which the reference's Triton kernel (fp8_linear.py:66-80) spells with a
 * clamp to +-448 that cannot trigger for finite rows. */
struct qrows { const uint16_t *x; int64_t K, ldx, ldy; uint8_t *y; float *s; };

static void qrows_body(void *p, int64_t r0, int64_t r1)
{
    struct qrows *c = p;
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t *xr = c->x + r * c->ldx;
        float amax = 0.0f;
        for (int64_t k = 0; k < c->K; ++k) amax = nanmax(amax, fabsf(oracle_bf16_to_f32(xr[k])));
        float scale = clamp_floor(amax / 448.0f);
        c->s[r] = scale;
        uint8_t *yr = c->y + r * c->ldy;
        for (int64_t k = 0; k < c->K; ++k) yr[k] = oracle_e4m3_from_f32(oracle_bf16_to_f32(xr[k]) / scale);
    }
}

void oracle_quantize_rows(const uint16_t *x, int64_t M, int64_t K, int64_t ldx,
                          uint8_t *y, int64_t ldy, float *scale, int nthreads)
{
    struct qrows c = {x, K, ldx, ldy, y, scale};
    parallel_rows(qrows_body, &c, M, nthreads);
}

/* ------------------------------------------------------------------------ */
/* fused SwiGLU + per-token quantization                                     */
/* ------------------------------------------------------------------------ */

/* Restates _swiglu_quantize_kernel (fp8_linear.py:83-99): for a row of h
 * [M, 2K], a = h[:, :K], g = h[:, K:], act = a * g * sigmoid(g) in fp32 (the
 * bf16 activation is never rounded), then the quantize_rows arithmetic on act.
 * sigmoid is 1 / (1 + exp(-g)) with libm's expf; kernels using another exp are
 * compared within one fp8 code. */
struct qswiglu { const uint16_t *h; int64_t K, ldh, ldy; uint8_t *y; float *s; };

static inline float swiglu_act(float a, float g) { return a * g * (1.0f / (1.0f + expf(-g))); }

static void qswiglu_body(void *p, int64_t r0, int64_t r1)
{
    struct qswiglu *c = p;
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t *hr = c->h + r * c->ldh;
        float amax = 0.0f;
        for (int64_t k = 0; k < c->K; ++k)
            amax = nanmax(amax, fabsf(swiglu_act(oracle_bf16_to_f32(hr[k]), oracle_bf16_to_f32(hr[c->K + k]))));
        float scale = clamp_floor(amax / 448.0f);
        c->s[r] = scale;
        uint8_t *yr = c->y + r * c->ldy;
        for (int64_t k = 0; k < c->K; ++k)
            yr[k] = oracle_e4m3_from_f32(swiglu_act(oracle_bf16_to_f32(hr[k]), oracle_bf16_to_f32(hr[c->K + k])) / scale);
    }
}

void oracle_swiglu_quantize_rows(const uint16_t *h, int64_t M, int64_t K, int64_t ldh,
                                 uint8_t *y, int64_t ldy, float *scale, int nthreads)
{
    struct qswiglu c = {h, K, ldh, ldy, y, scale};
    parallel_rows(qswiglu_body, &c, M, nthreads);
}

/* ------------------------------------------------------------------------ */
/* rowwise weight quantization (Fp8Linear.__init__)                          */
/* ------------------------------------------------------------------------ */

/* Restates the rowwise branch of Fp8Linear.__init__ (fp8_linear.py:262-267):
 *   scale = (weight.abs().amax(dim=1, keepdim=True).float() / 448).clamp_min(1e-12)
 *   weight_fp8 = (weight / scale.to(weight.dtype)).to(float8_e4m3fn)
 *   weight_scale = scale.reshape(1, -1)              # the fp32 scale is stored
 * weight / bf16_scale is a bf16 / bf16 division: binary32 quotient rounded to
 * bf16, then cast to e4m3 -- two roundings that the codes must reproduce. */
struct qweight { const uint16_t *w; int64_t K, ldw, ldq; uint8_t *q; float *s; };

static void qweight_body(void *p, int64_t r0, int64_t r1)
{
    struct qweight *c = p;
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t *wr = c->w + r * c->ldw;
        float amax = 0.0f;
        for (int64_t k = 0; k < c->K; ++k) amax = nanmax(amax, fabsf(oracle_bf16_to_f32(wr[k])));
        float scale = clamp_floor(amax / 448.0f);
        c->s[r] = scale;
        float sb = oracle_bf16_to_f32(oracle_bf16_from_f32(scale));
        uint8_t *qr = c->q + r * c->ldq;
        for (int64_t k = 0; k < c->K; ++k) {
            float quot = oracle_bf16_to_f32(oracle_bf16_from_f32(oracle_bf16_to_f32(wr[k]) / sb));
            qr[k] = oracle_e4m3_from_f32(quot);
        }
    }
}

void oracle_quantize_weight(const uint16_t *w, int64_t N, int64_t K, int64_t ldw,
                            uint8_t *q, int64_t ldq, float *scale, int nthreads)
{
    struct qweight c = {w, K, ldw, ldq, q, scale};
    parallel_rows(qweight_body, &c, N, nthreads);
}

/* ------------------------------------------------------------------------ */
/* LoRA merge                                                                */
/* ------------------------------------------------------------------------ */

/* Restates merge_lora_state's update (inference/utils/lora.py:91-92):
 *   delta = (b.to(float32) @ a.to(float32)) * scale
 *   w.data.add_(delta.to(w.dtype))
 * with b bf16 [N, r], a bf16 [r, K], w bf16 [N, K].  The reference leaves the
 * fp32 summation order to the BLAS; products of bf16 values are exact in
 * binary32, so the oracle sums them in binary64 and rounds once to binary32 --
 * the value every fp32 summation order approximates to within a few binary32
 * ulps.  Then the binary32 multiply by scale, the bf16 rounding of delta, and
 * the bf16 add (binary32 add rounded to bf16). */
struct lmerge { const uint16_t *w, *a, *b; int64_t K, r, ldw, ldo; float scale; uint16_t *out; };

static void lmerge_body(void *p, int64_t n0, int64_t n1)
{
    struct lmerge *c = p;
    for (int64_t n = n0; n < n1; ++n) {
        for (int64_t k = 0; k < c->K; ++k) {
            double acc = 0.0;
            for (int64_t j = 0; j < c->r; ++j)
                acc += (double)oracle_bf16_to_f32(c->b[n * c->r + j]) * (double)oracle_bf16_to_f32(c->a[j * c->K + k]);
            float delta = (float)acc * c->scale;
            float d16 = oracle_bf16_to_f32(oracle_bf16_from_f32(delta));
            float w = oracle_bf16_to_f32(c->w[n * c->ldw + k]);
            c->out[n * c->ldo + k] = oracle_bf16_from_f32(w + d16);
        }
    }
}

void oracle_lora_merge(const uint16_t *w, int64_t N, int64_t K, int64_t ldw,
                       const uint16_t *a, const uint16_t *b, int64_t r, float scale,
                       uint16_t *out, int64_t ldo, int nthreads)
{
    struct lmerge c = {w, a, b, K, r, ldw, ldo, scale, out};
    parallel_rows(lmerge_body, &c, N, nthreads);
}

/* ------------------------------------------------------------------------ */
/* batch element-wise entry points (for the pinning tests)                   */
/* ------------------------------------------------------------------------ */

void oracle_e4m3_encode(const float *x, int64_t n, uint8_t *y)
{
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_e4m3_from_f32(x[i]);
}

void oracle_e4m3_decode(const uint8_t *c, int64_t n, float *y)
{
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_e4m3_to_f32(c[i]);
}

void oracle_bf16_encode(const float *x, int64_t n, uint16_t *y)
{
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_bf16_from_f32(x[i]);
}

int oracle_version(void) { return 1; }
