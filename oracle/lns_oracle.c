/*
 * lns_oracle.c - CPU restatement of the reference LNS16/LNS32 CPU backend.
 *
 * TEST INFRASTRUCTURE ONLY (see lns_oracle.h).  Single-threaded on purpose:
 * the reference backend is single-threaded (lns-backend/common/
 * lns-backend-framework.h:207-221) and its Monte LFSR is one process-global
 * state (src/lns-ops.cpp:155-195).
 *
 * The arithmetic library the reference compiles in (xlnscpp, pinned
 * 41843b0, patches/xlnscpp-base-commit.txt:1) is an empty submodule in the
 * reference checkout.  What follows restates its published algorithm as the
 * reference configures it; each block names what pins it.
 *
 * Parity status (tests/test_oracle_pins.py, tests/test_reference_figures.py):
 *   xlns16 codes, mul, div, recip, widen/narrow ......... pinned (closed form,
 *       unit-tests-lns16-base.txt div/clamp values, exhaustive round trip)
 *   fp2xlns16 table / xlns162fp ........................... pinned: known codes of
 *       unit-tests-lns16-base.txt; all eleven statistics of convert.jsonl:1
 *       to six digits, over the experiment's own 4M operands
 *   xlns16_add (sb/db table, xlns16_alt) ................ pinned: stagnation
 *       codes 897/1092, two-term statistics, the base K=2, K=1536,
 *       mul_mat_id, soft_max and rms_norm figures of unit-tests-lns16-base.txt,
 *       and every base row of synth.jsonl (K = 16..16384, three operand
 *       distributions, five statistics to six digits)
 *   sqrt, exp table, softmax/rms_norm drivers ........... pinned by the same
 *       base and sum32 figures
 *   xlns32_add (xlns32_alt) ............................. parity contradicted in
 *       part: reproduces 28 of the 31 xlns32-dependent unit-test and
 *       standalone figures; misses standalone K=8960 (0.211% vs 0.198%),
 *       LNS32 K=1536 (NRMSE 0.0124% vs 0.0122%) and LNS32 mul_mat_id
 *       broadcast (0.0000% vs 0.0001%).  The experiment's xlns32 rows came
 *       from a different (post-merge) adder whose sb is recovered exactly
 *       (lno32_set_variant(1)) and which cannot be the unit-test one
 *   fp2xlns32 / xlns322fp ................................ pinned: all eleven
 *       statistics of convert.jsonl:2 to six digits
 *   monte (xlns16_add_monte) ............................. parity contradicted
 *       in part: the xlnscpp source is absent; the restatement, fitted to
 *       the printed figures, reproduces 13 of the 15 monte unit-test
 *       figures and no synth.jsonl row (the LFSR itself is pinned)
 *   lpvip (xlns32_add_lpvip) ............................. parity contradicted:
 *       the xlnscpp source is absent and this restatement misses the
 *       reference's printed figures
 *   expf-based xlns32 exp, xlns32_silu .................. parity unpinned below
 *       the six printed digits
 */
#include "lns_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * xlns16 format (src/lns16-sum32.h:52-81, tests/test-lns16-sum32.cpp:37-52):
 * bit 15 sign, bits 14..0 = 128*log2|x| + 0x4000; 0x0000 is zero.
 * ==================================================================== */
#define X16_SIGN     0x8000u
#define X16_LOGMASK  0x7fffu
#define X16_ONE      0x4000u   /* also the log offset ("logsignmask") */
#define X16_SQRTMASK 0x2000u
#define X16_ESSZER   1280      /* 0x0500: beyond this distance an addend is dropped */
#define X16_NEG_INF  0xffffu   /* largest-magnitude negative value */

static uint16_t g_cvt16[1u << 17];   /* float bits >> 15  ->  xlns16 */
static float    g_rev16[1u << 16];   /* xlns16 -> float */
static int16_t  g_sb16[X16_ESSZER + 1];
static int16_t  g_db16[X16_ESSZER + 1];
static uint16_t g_exp16[1u << 16];
static uint16_t g_sig16[1u << 16];
static int      g_ready = 0;

static inline float f32_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t bits_from_f32(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* The value an x86-64 compiler gives for (int16_t)(double): the double is
 * truncated to a 32-bit integer (0x80000000 when out of range or NaN) and the
 * low 16 bits are kept. */
static inline int16_t trunc_to_s16(double v) {
    int32_t i;
    if (!(v > -2147483649.0 && v < 2147483648.0)) i = INT32_MIN;
    else i = (int32_t)v;
    return (int16_t)(uint16_t)(uint32_t)i;
}
static inline int32_t trunc_to_s32(double v) {
    if (!(v > -2147483649.0 && v < 2147483648.0)) return INT32_MIN;
    return (int32_t)v;
}

/* xlnscpp's direct (non-table) float -> xlns16: the log is truncated toward
 * zero, then offset by xor with 0x4000. */
static uint16_t fp2xlns16_direct(float x) {
    if (x == 0.0f) return 0;
    if (x > 0.0f) {
        int16_t l = trunc_to_s16((log((double)x) / log(2.0)) * 128.0);
        return (uint16_t)(((uint16_t)l & X16_LOGMASK) ^ X16_ONE);
    }
    int16_t l = trunc_to_s16((log(fabs((double)x)) / log(2.0)) * 128.0);
    return (uint16_t)(((uint16_t)l | X16_SIGN) ^ X16_ONE);
}

/* xlnscpp's direct xlns16 -> float. */
static float xlns162fp_direct(uint16_t v) {
    if ((v & X16_LOGMASK) == 0) return 0.0f;
    double l = (double)(int16_t)(uint16_t)((v & X16_LOGMASK) - X16_ONE) / 128.0;
    double m = pow(2.0, l);
    return (float)((v & X16_SIGN) ? -m : m);
}

/* The xlns16 -> float table holds each value as a decimal literal with 7
 * significant digits ("%e" of the float), read back as a float: 2^(1355/128)
 * decodes to 1537.0380 and 2^(491/128) to 14.280130, as the reference prints
 * them (standalone-sum32-invariants.txt:10, unit-tests-lns16-base.txt:29). */
static float rev16_entry(uint16_t v) {
    float f = xlns162fp_direct(v);
    if (f == 0.0f) return f;
    char buf[64];
    snprintf(buf, sizeof buf, "%e", (double)f);
    return (float)strtod(buf, NULL);
}

uint16_t lno16_mul(uint16_t x, uint16_t y) {
    uint16_t t = (uint16_t)((x & X16_LOGMASK) + (y & X16_LOGMASK) - X16_ONE);
    uint16_t s = (uint16_t)((x ^ y) & X16_SIGN);
    if (t & X16_SIGN) return (t & X16_ONE) ? s : (uint16_t)(s | X16_LOGMASK);
    return (uint16_t)(s | t);
}

uint16_t lno16_div(uint16_t x, uint16_t y) {
    uint16_t t = (uint16_t)((x & X16_LOGMASK) - (y & X16_LOGMASK) + X16_ONE);
    uint16_t s = (uint16_t)((x ^ y) & X16_SIGN);
    if (t & X16_SIGN) return (t & X16_ONE) ? s : (uint16_t)(s | X16_LOGMASK);
    return (uint16_t)(s | t);
}

/* log field halved, rounding half away from zero; sign dropped */
uint16_t lno16_sqrt(uint16_t x) {
    int16_t sh = (int16_t)(uint16_t)(x << 1);
    int q = sh / 4;
    return (uint16_t)(((unsigned)q & X16_LOGMASK) ^ X16_SQRTMASK);
}

uint16_t lno16_recip(uint16_t x) {
    return (uint16_t)((x & X16_SIGN) | ((uint16_t)(~x + 1u) & X16_LOGMASK));
}

/* canonical order: negative values get their log bits flipped, then the
 * code compares as a signed 16-bit integer */
static inline int16_t canon16(uint16_t x) {
    return (int16_t)(uint16_t)((x & X16_SIGN) ? (x ^ X16_LOGMASK) : x);
}
int lno16_gt(uint16_t a, uint16_t b) { return canon16(a) > canon16(b); }

/* Gaussian logs at integer distance d = max - min >= 0, as xlnscpp's
 * xlns16_alt adder forms them (x + (int)(log2(+-1 + 2^(d/128))*128 + .5)). */
static int16_t sb16_entry(int d) {
    double v = log(1.0 + pow(2.0, (double)d / 128.0)) / log(2.0) * 128.0 + 0.5;
    return (int16_t)(-d + (int)trunc_to_s32(v));
}
static int16_t db16_entry(int d) {
    double v = log(-1.0 + pow(2.0, (double)d / 128.0)) / log(2.0) * 128.0 + 0.5;
    return (int16_t)(-d + (int)trunc_to_s32(v));
}

/* xlns16_add with xlns16_alt: the larger operand scaled by 2^(adjust/128) */
uint16_t lno16_add(uint16_t x, uint16_t y) {
    unsigned xl = x & X16_LOGMASK, yl = y & X16_LOGMASK;
    unsigned minl = yl > xl ? xl : yl;
    uint16_t maxxy = xl > yl ? x : y;
    int z = (int)minl - (int)(maxxy & X16_LOGMASK);
    int usedb = ((x ^ y) & X16_SIGN) != 0;
    if (z == 0 && usedb) return 0;
    int adj = 0;
    if (z >= -X16_ESSZER) adj = usedb ? g_db16[-z] : g_sb16[-z];
    return lno16_mul(maxxy, (uint16_t)(X16_ONE + adj));
}

uint16_t lno16_sub(uint16_t x, uint16_t y) { return lno16_add(x, (uint16_t)(y ^ X16_SIGN)); }

uint16_t lno16_exp(uint16_t x) { return g_exp16[x]; }

/* xlns16_silu: x * sigmoid(x), the sigmoid through the bucketed conversion
 * table.  Pinned by the eight swiglu values of unit-tests-lns16-base.txt
 * (test-lns-backend.cpp:554-580 inputs); the alternatives miss one to four. */
uint16_t lno16_silu(uint16_t x) { return lno16_mul(x, g_sig16[x]); }

uint16_t lno16_from_f32(float x) { return g_cvt16[bits_from_f32(x) >> 15]; }
float    lno16_to_f32(uint16_t v) { return g_rev16[v]; }

void lno16_from_f32_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = lno16_from_f32(src[i]);
}
void lno16_to_f32_n(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = lno16_to_f32(src[i]);
}

const uint16_t *lno16_cvt_table(void) { return g_cvt16; }
const int16_t  *lno16_sb_table(void)  { return g_sb16; }
const int16_t  *lno16_db_table(void)  { return g_db16; }
const uint16_t *lno16_exp_table(void) { return g_exp16; }

/* ======================================================================
 * sum32 accumulator (src/lns16-sum32.h:59-81): exact widening into xlns32,
 * one round-half-up narrowing with saturation.
 * ==================================================================== */
uint32_t lno16_widen(uint16_t v) { return (uint32_t)v << 16; }

uint16_t lno16_narrow_sum32(uint32_t s) {
    if ((s & 0x7fffffffu) >= 0x7fff8000u) return (uint16_t)((s >> 16) | X16_LOGMASK);
    return (uint16_t)((s + 0x8000u) >> 16);
}

/* lpvip narrows by truncation (src/lns16-sum32.h:63-66) */
uint16_t lno16_narrow_lpvip(uint32_t s) { return (uint16_t)(s >> 16); }

/* ======================================================================
 * xlns32 (README.md:144-147): bit 31 sign, bits 30..0 = 2^23*log2|x| +
 * 0x40000000.  Addition follows xlns32_alt: sb by table + linear
 * interpolation, db by cotransformation near the singularity.
 * ==================================================================== */
#define X32_SIGN    0x80000000u
#define X32_LOGMASK 0x7fffffffu
#define X32_ONE     0x40000000u
#define X32_SQRTMASK 0x20000000u
#define X32_NEG_INF 0xffffffffu
#define X32_ESSZER  (24 << 23)      /* 24 binades */

/* xlns32_alt's tables are not published.  This grid and rounding are the
 * ones, among the natural candidates tried, that reproduce the reference's
 * printed xlns32-accumulator figures: sums of ones to 8960 and 65536
 * (codes 1680 and 2048, standalone-sum32-invariants.txt:8-11), the sum32
 * K=1536 dot statistics (:13), the sum32 K=1536 NRMSE 0.3075% and max
 * 0.8116% (unit-tests-lns16-sum32.txt:12-14) and the LNS32 rms_norm 576
 * error 0.0012% (unit-tests-lns32.txt:131).  Near misses: LNS32 K=1536
 * NRMSE 0.0124% vs 0.0122%, sum32 K=8960 mean 0.211% vs 0.198%.
 *
 *   sb(d)  = log2(1 + 2^-d):  nodes every 2^13 below 12 binades, every
 *            2^19 from 12 to 24 binades; entries truncated
 *   db(d)  = log2(1 - 2^-d):  nodes every 2^13 from 2 to 8 binades, every
 *            2^19 from 8 to 24 binades; entries floored
 *   both:  linear interpolation between nodes, floored
 *   db below 2 binades: cotransformation d = dh + dl with dl the low 12
 *            bits, from two floored tables (db at dl, db at dh) and sb. */
#define X32_SB_END  (12 << 23)
#define X32_SB_SH   13
#define X32_SB_FSH  19
#define X32_DB_END  (8 << 23)
#define X32_DB_SH   13
#define X32_DB_FSH  19
#define X32_CO_END  (1 << 24)
#define X32_CO_SH   12
#define X32_SB_N    (X32_SB_END >> X32_SB_SH)
#define X32_SB_FN   ((X32_ESSZER - X32_SB_END) >> X32_SB_FSH)
#define X32_DB_N    (X32_DB_END >> X32_DB_SH)
#define X32_DB_FN   ((X32_ESSZER - X32_DB_END) >> X32_DB_FSH)

static int32_t g_sb32a[X32_SB_N + 1], g_sb32b[X32_SB_FN + 1];
static int32_t g_db32a[X32_DB_N + 1], g_db32b[X32_DB_FN + 1];
static int32_t g_db32lo[1 << X32_CO_SH];               /* db at d = dl      */
static int32_t g_db32hi[X32_CO_END >> X32_CO_SH];      /* db at d = i*4096  */

static long double sb32_exact(long double d) { return log2l(1.0L + exp2l(-d / 8388608.0L)) * 8388608.0L; }
static long double db32_exact(long double d) { return log2l(1.0L - exp2l(-d / 8388608.0L)) * 8388608.0L; }

static int32_t interp32(const int32_t *ta, const int32_t *tb, uint32_t d, uint32_t aend, int ash, int bsh) {
    const int32_t *t = ta;
    int sh = ash;
    if (d >= aend) {
        t = tb;
        sh = bsh;
        d -= aend;
    }
    uint32_t i = d >> sh, f = d & ((1u << sh) - 1);
    int32_t t0 = t[i], t1 = t[i + 1];
    return t0 + (int32_t)(((int64_t)(t1 - t0) * (int64_t)f) >> sh);
}

/* The xlns32 sb that the reference's experiments ran with (post-merge
 * xlnscpp 4f5e75f + PR #64 and xlnscuda f0834bb + PR #11,
 * experiments/README.md:28-37): one grid of nodes every 2^14 up to 24
 * binades, entries floored, linear interpolation rounded to nearest.  It
 * reproduces every positive-operand xlns32 row of
 * experiments/dot-product-scaling/results/synth.jsonl (K = 16..16384) to
 * all six printed digits, where only sb runs.  It is NOT the sb of the
 * unit-test evidence: it sums 8960 ones to code 1681, where
 * standalone-sum32-invariants.txt:10 prints code 1680 (8933.4395).  Tests
 * select it with lno32_set_variant(1) to show that the two evidence sets
 * come from different adders; the op drivers never use it otherwise. */
#define X32_PM_SH 14
static int32_t g_sb32pm[(X32_ESSZER >> X32_PM_SH) + 2];
static int g_x32_variant = 0;

static int32_t sb32_postmerge(uint32_t d) {     /* d < X32_ESSZER */
    uint32_t i = d >> X32_PM_SH, f = d & ((1u << X32_PM_SH) - 1);
    int64_t t0 = g_sb32pm[i], t1 = g_sb32pm[i + 1];
    return (int32_t)(t0 + (((t1 - t0) * (int64_t)f + (1 << (X32_PM_SH - 1))) >> X32_PM_SH));
}

int lno32_set_variant(int v) {
    if (v != 0 && v != 1) return -1;
    int old = g_x32_variant;
    g_x32_variant = v;
    return old;
}

static int32_t sb32(uint32_t d) {               /* d < X32_ESSZER */
    if (g_x32_variant == 1) return sb32_postmerge(d);
    return interp32(g_sb32a, g_sb32b, d, (uint32_t)X32_SB_END, X32_SB_SH, X32_SB_FSH);
}

static int32_t db32(uint32_t d) {               /* 0 < d < X32_ESSZER */
    if (d >= (uint32_t)X32_CO_END) return interp32(g_db32a, g_db32b, d, (uint32_t)X32_DB_END, X32_DB_SH, X32_DB_FSH);
    uint32_t dl = d & ((1u << X32_CO_SH) - 1), dh = d - dl;
    if (dh == 0) return g_db32lo[dl];
    int32_t th = g_db32hi[dh >> X32_CO_SH];
    if (dl == 0) return th;
    /* 1 - 2^-d = (1 - 2^-dh) + 2^-dh (1 - 2^-dl) */
    int32_t w = -(int32_t)dh + g_db32lo[dl] - th;  /* < 0 */
    uint32_t e = (uint32_t)(-w);
    return th + (e < (uint32_t)X32_ESSZER ? sb32(e) : 0);
}

uint32_t lno32_mul(uint32_t x, uint32_t y) {
    uint32_t t = (x & X32_LOGMASK) + (y & X32_LOGMASK) - X32_ONE;
    uint32_t s = (x ^ y) & X32_SIGN;
    if (t & X32_SIGN) return (t & X32_ONE) ? s : (s | X32_LOGMASK);
    return s | t;
}

uint32_t lno32_div(uint32_t x, uint32_t y) {
    uint32_t t = (x & X32_LOGMASK) - (y & X32_LOGMASK) + X32_ONE;
    uint32_t s = (x ^ y) & X32_SIGN;
    if (t & X32_SIGN) return (t & X32_ONE) ? s : (s | X32_LOGMASK);
    return s | t;
}

uint32_t lno32_add(uint32_t x, uint32_t y) {
    uint32_t xl = x & X32_LOGMASK, yl = y & X32_LOGMASK;
    uint32_t minl = yl > xl ? xl : yl;
    uint32_t maxxy = xl > yl ? x : y;
    uint32_t d = (maxxy & X32_LOGMASK) - minl;
    int usedb = ((x ^ y) & X32_SIGN) != 0;
    if (d == 0 && usedb) return 0;
    int32_t adj = 0;
    if (d < (uint32_t)X32_ESSZER) adj = usedb ? db32(d) : sb32(d);
    return lno32_mul(maxxy, X32_ONE + (uint32_t)adj);
}

uint32_t lno32_sub(uint32_t x, uint32_t y) { return lno32_add(x, y ^ X32_SIGN); }

/* the interpolation / cotransformation tables, for tests */
const int32_t *lno32_table(const char *name, size_t *n) {
    struct { const char *k; const int32_t *p; size_t n; } t[] = {
        {"sb", g_sb32a, X32_SB_N + 1}, {"sbf", g_sb32b, X32_SB_FN + 1},
        {"db", g_db32a, X32_DB_N + 1}, {"dbf", g_db32b, X32_DB_FN + 1},
        {"dlo", g_db32lo, 1 << X32_CO_SH}, {"dhi", g_db32hi, X32_CO_END >> X32_CO_SH},
    };
    for (size_t i = 0; i < sizeof t / sizeof t[0]; i++)
        if (strcmp(t[i].k, name) == 0) { *n = t[i].n; return t[i].p; }
    *n = 0;
    return NULL;
}

uint32_t lno32_sqrt(uint32_t x) {
    int32_t sh = (int32_t)(x << 1);
    int32_t q = sh / 4;
    return ((uint32_t)q & X32_LOGMASK) ^ X32_SQRTMASK;
}

uint32_t lno32_recip(uint32_t x) { return (x & X32_SIGN) | ((~x + 1u) & X32_LOGMASK); }

static inline int32_t canon32(uint32_t x) {
    return (int32_t)((x & X32_SIGN) ? (x ^ X32_LOGMASK) : x);
}
int lno32_gt(uint32_t a, uint32_t b) { return canon32(a) > canon32(b); }

/* float -> xlns32: truncation toward zero of 2^23*log2|x| (correctly
 * evaluated), offset by xor with 0x40000000.  Denormals wrap exactly as
 * the 31-bit field arithmetic does. */
uint32_t lno32_from_f32(float x) {
    if (x == 0.0f) return 0;
    if (isnan(x)) return 0x80000000u ^ X32_ONE;
    uint32_t b = bits_from_f32(x);
    uint32_t s = b & 0x80000000u;
    if (isinf(x)) return s ? (0x80000000u ^ X32_ONE) : X32_ONE;
    long double l = log2l(fabsl((long double)x)) * 8388608.0L;
    int64_t t = (int64_t)l;  /* toward zero */
    uint32_t li = (uint32_t)(int32_t)t;
    if (!s) return (li & X32_LOGMASK) ^ X32_ONE;
    return (li | X32_SIGN) ^ X32_ONE;
}

float lno32_to_f32(uint32_t v) {
    if ((v & X32_LOGMASK) == 0) return 0.0f;
    long double l = (long double)(int32_t)((v & X32_LOGMASK) - X32_ONE) / 8388608.0L;
    long double m = exp2l(l);
    float f = (float)m;
    return (v & X32_SIGN) ? -f : f;
}

void lno32_from_f32_n(const float *src, uint32_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = lno32_from_f32(src[i]);
}
void lno32_to_f32_n(const uint32_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = lno32_to_f32(src[i]);
}

/* xlns32 exp goes through float expf (docs/CUDA.md:159-161); evaluated here
 * correctly rounded. */
uint32_t lno32_exp(uint32_t x) {
    float v = lno32_to_f32(x);
    float e = (float)expl((long double)v);
    return lno32_from_f32(e);
}

/* ======================================================================
 * Monte LFSR (src/lns-ops.cpp:178-195): 16-bit Galois LFSR, taps 0xB400,
 * period 65535, seed 7; state 0 is absorbing and rejected.
 * ==================================================================== */
static uint16_t g_lfsr = 7;
static uint16_t g_lfsr_seq[65535];   /* state after i steps from state 1 */
static uint16_t g_lfsr_log[65536];   /* inverse of g_lfsr_seq */

uint16_t lno_lfsr_step(uint16_t s) {
    uint16_t bit = s & 1u;
    s >>= 1;
    if (bit) s ^= 0xB400u;
    return s;
}

uint16_t lno_lfsr_jump(uint16_t s, uint64_t n) {
    if (s == 0) return 0;
    uint32_t i = g_lfsr_log[s];
    return g_lfsr_seq[(uint32_t)((i + n % 65535u) % 65535u)];
}

int lno_monte_get_state(uint16_t *state) { *state = g_lfsr; return 1; }
int lno_monte_set_state(uint16_t state) {
    if (state == 0) return 0;
    g_lfsr = state;
    return 1;
}
int lno_monte_reserve(uint64_t draws, uint16_t *start) {
    *start = g_lfsr;
    g_lfsr = lno_lfsr_jump(g_lfsr, draws);
    return 1;
}

/* ======================================================================
 * Monte addition (xlns16monte.cpp, pure16; src/lns-ops.cpp:86-98).  One
 * LFSR step per addition (src/lns-ops.cpp:178-195 counts one draw per add).
 * The library is absent; this restatement is fitted to the reference's
 * printed figures.  What they fix structurally:
 *   - every K <= 8 sum of the monte unit tests printed the base value
 *     (unit-tests-lns16-monte.txt:4-7, :17-26), so additions at moderate
 *     distances are the deterministic xlns16_add;
 *   - the dither acts where xlns16_add's Gaussian log rounds to 0 (sums
 *     stagnate there: src/lns16-sum32.h:3-6): monte's positive-operand
 *     bias in synth.jsonl is +8 % at K = 1024 where base loses 20 %;
 *   - the dither is a draw of +-1 ulp: synth.jsonl's monte sd follows a
 *     random walk of unit steps, and with the LFSR's high bits (not its
 *     low bits, which repeat shifted from one draw to the next) the sd
 *     of every positive row (K = 16..16384) comes out within 2 %.
 * Fitted: from distance 1091 on (where the exact sb is 0.501 ulp), the
 * addition moves the larger log by one ulp toward the smaller operand with
 * probability F(d)/64, F(d) = floor(2^(-d/128) * 185 * 64) (the first-order
 * sb, 128/ln 2 = 184.7, at 6 bits), decided by the top 6 bits of the new
 * LFSR state: adj = +-((F(d) + (r >> 10)) >> 6).  F is 0 from d = 1732 on.
 * This reproduces 13 of the 15 printed monte unit-test figures (K = 2,
 * the four mul_mat_id cases, both rms_norm cases, the K = 1536 maximum,
 * four of five soft_max cases) and misses two: K = 1536 NRMSE (4.9245 %
 * vs 4.7150 %) and soft_max masked_scaled (0.000287 vs 0.000494).  It
 * matches no synth.jsonl row to six digits.  Parity contradicted.
 * ==================================================================== */
#define X16_MC_START 1091
#define X16_MC_END   1732      /* F(d) = 0 from here on */
static int32_t g_mc16[X16_MC_END + 1];

uint16_t lno16_add_monte(uint16_t x, uint16_t y, uint16_t *lfsr) {
    uint16_t r = lno_lfsr_step(*lfsr);
    *lfsr = r;
    unsigned xl = x & X16_LOGMASK, yl = y & X16_LOGMASK;
    unsigned minl = yl > xl ? xl : yl;
    uint16_t maxxy = xl > yl ? x : y;
    int z = (int)minl - (int)(maxxy & X16_LOGMASK);
    int usedb = ((x ^ y) & X16_SIGN) != 0;
    if (z == 0 && usedb) return 0;
    int d = -z, adj;
    if (d < X16_MC_START) {
        adj = usedb ? g_db16[d] : g_sb16[d];
    } else {
        int32_t f = d < X16_MC_END ? g_mc16[d] : 0;
        int32_t m = (f + (int32_t)(r >> 10)) >> 6;
        adj = usedb ? -m : m;
    }
    return lno16_mul(maxxy, (uint16_t)(X16_ONE + adj));
}

/* the dither threshold F(d) at d0 .. d0 + n - 1 (0 outside the dither range) */
void lno16_monte_threshold_n(int d0, int n, int32_t *out) {
    for (int i = 0; i < n; i++) {
        int d = d0 + i;
        out[i] = (d >= X16_MC_START && d < X16_MC_END) ? g_mc16[d] : 0;
    }
}

/* ======================================================================
 * LPVIP accumulator (xlns32lpvip.cpp): a ROM-less xlns32 adder.  sb is a
 * Mitchell antilog followed by a Mitchell log; db uses the same pair away
 * from the singularity and the exact Gaussian log (double log/pow) within
 * one binade of it.  Terms are widened exactly, the result is truncated.
 * parity unpinned (see file header).
 * ==================================================================== */
static uint32_t mitchell_exp2_neg(uint32_t d) {  /* ~2^(-d/2^23) * 2^23 */
    uint32_t q = d >> 23, r = d & 0x7fffffu;
    if (q >= 31) return 0;
    /* 2^(-r) = 2^(1-r)/2 ~ (2 - r)/2 */
    return ((0x1000000u - r) >> 1) >> q;
}
static int32_t lpvip_sb(uint32_t d) {            /* log2(1 + u) ~ u, corrected */
    uint32_t u = mitchell_exp2_neg(d);
    /* Mitchell log: log2(1+u) ~ u + u(1-u)*0.34 (one-term correction) */
    uint64_t corr = ((uint64_t)u * (uint64_t)(0x800000u - u)) >> 23;
    return (int32_t)(u + (uint32_t)((corr * 0x2B8u) >> 11));
}
static int32_t lpvip_db_exact(uint32_t d) {
    double v = log(1.0 - pow(2.0, -(double)d / 8388608.0)) / log(2.0) * 8388608.0;
    return (int32_t)floor(v + 0.5);
}
static int32_t lpvip_db(uint32_t d) {
    if (d < 0x800000u) return lpvip_db_exact(d);
    /* log2(1 - u) ~ -(u + u^2/2 * 1.44) */
    uint32_t u = mitchell_exp2_neg(d);
    uint64_t sq = ((uint64_t)u * u) >> 23;
    return -(int32_t)(u + (uint32_t)((sq * 0xB8Au) >> 12));
}

/* lpvip db at d for d0 .. d0 + n - 1 (the checker of the GPU's db) */
void lno32_lpvip_db_n(uint32_t d0, uint32_t n, int32_t *out) {
    for (uint32_t i = 0; i < n; i++) out[i] = lpvip_db(d0 + i);
}

uint32_t lno16_lpvip_add(uint32_t acc, uint16_t t16) {
    uint32_t t = lno16_widen(t16);
    uint32_t al = acc & X32_LOGMASK, tl = t & X32_LOGMASK;
    uint32_t minl = tl > al ? al : tl;
    uint32_t maxxy = al > tl ? acc : t;
    uint32_t d = (maxxy & X32_LOGMASK) - minl;
    int usedb = ((acc ^ t) & X32_SIGN) != 0;
    if (d == 0 && usedb) return 0;
    int32_t adj = 0;
    if (d < (uint32_t)X32_ESSZER) adj = usedb ? lpvip_db(d) : lpvip_sb(d);
    return lno32_mul(maxxy, X32_ONE + (uint32_t)adj);
}

/* ======================================================================
 * Reductions.  Term orders follow the reference GPU mirror, which is
 * bit-identical to the CPU in every mode (cuda/lns-cuda-kernels.cuh):
 *   vec_dot: acc = a0*b0, then += ak*bk for k = 1..n-1   (:110-152)
 *   sum:     acc = a0, then += ak for k = 1..n-1          (:311-319)
 *   rms:     acc = zero, then += xk^2 for k = 0..n-1      (:235-243)
 * ==================================================================== */
typedef struct { int mode; uint16_t *lfsr; uint32_t acc; } red16;

static inline void red_start(red16 *r, uint16_t v) {
    r->acc = (r->mode == LNO_SUM32 || r->mode == LNO_LPVIP) ? lno16_widen(v) : v;
}
static inline void red_add(red16 *r, uint16_t t) {
    switch (r->mode) {
        case LNO_SUM32: r->acc = lno32_add(r->acc, lno16_widen(t)); break;
        case LNO_LPVIP: r->acc = lno16_lpvip_add(r->acc, t); break;
        case LNO_MONTE: r->acc = lno16_add_monte((uint16_t)r->acc, t, r->lfsr); break;
        default:        r->acc = lno16_add((uint16_t)r->acc, t); break;
    }
}
static inline uint16_t red_finish(const red16 *r) {
    switch (r->mode) {
        case LNO_SUM32: return lno16_narrow_sum32(r->acc);
        case LNO_LPVIP: return lno16_narrow_lpvip(r->acc);
        default:        return (uint16_t)r->acc;
    }
}

uint16_t lno16_sum(int mode, const uint16_t *a, size_t n, uint16_t *lfsr) {
    if (n == 0) return 0;
    red16 r = { mode, lfsr ? lfsr : &g_lfsr, 0 };
    red_start(&r, a[0]);
    for (size_t i = 1; i < n; i++) red_add(&r, a[i]);
    return red_finish(&r);
}

uint16_t lno16_vec_dot(int mode, const uint16_t *a, const uint16_t *b, size_t n, uint16_t *lfsr) {
    if (n == 0) return 0;
    red16 r = { mode, lfsr ? lfsr : &g_lfsr, 0 };
    red_start(&r, lno16_mul(a[0], b[0]));
    for (size_t i = 1; i < n; i++) red_add(&r, lno16_mul(a[i], b[i]));
    return red_finish(&r);
}

/* src/lns16-sum32.h:142-151 (and the same order for every mode) */
void lno16_rms_norm_row(int mode, const uint16_t *x, uint16_t *dst, size_t n, uint16_t eps, uint16_t *lfsr) {
    if (n == 0) return;
    red16 r = { mode, lfsr ? lfsr : &g_lfsr, 0 };
    red_start(&r, 0);
    for (size_t i = 0; i < n; i++) red_add(&r, lno16_mul(x[i], x[i]));
    uint16_t mean = lno16_mul(red_finish(&r), lno16_from_f32(1.0f / (float)n));
    uint16_t inv = lno16_recip(lno16_sqrt(lno16_add(mean, eps)));
    for (size_t i = 0; i < n; i++) dst[i] = lno16_mul(x[i], inv);
}

/* src/lns16-sum32.h:158-198 (and the same order for every mode) */
void lno16_softmax_row(int mode, const uint16_t *a, const uint16_t *mask, uint16_t *c, size_t n,
                       uint16_t scale, uint16_t *lfsr) {
    if (n == 0) return;
    uint16_t maxval = X16_NEG_INF;
    for (size_t i = 0; i < n; i++) {
        uint16_t v = a[i];
        if (v != X16_NEG_INF) {
            v = lno16_mul(v, scale);
            if (mask) {
                if (mask[i] == X16_NEG_INF) v = X16_NEG_INF;
                else if ((mask[i] & X16_LOGMASK) != 0) v = lno16_add(v, mask[i]);
            }
        }
        c[i] = v;
        if (lno16_gt(c[i], maxval)) maxval = c[i];
    }
    for (size_t i = 0; i < n; i++) c[i] = lno16_exp(lno16_sub(c[i], maxval));
    uint16_t total = lno16_sum(mode, c, n, lfsr);
    for (size_t i = 0; i < n; i++) c[i] = lno16_div(c[i], total);
}

/* xlns32 reductions (LNS32 backend: plain sequential xlns32_add) */
uint32_t lno32_vec_dot(const uint32_t *a, const uint32_t *b, size_t n) {
    if (n == 0) return 0;
    uint32_t acc = lno32_mul(a[0], b[0]);
    for (size_t i = 1; i < n; i++) acc = lno32_add(acc, lno32_mul(a[i], b[i]));
    return acc;
}

void lno32_rms_norm_row(const uint32_t *x, uint32_t *dst, size_t n, uint32_t eps) {
    if (n == 0) return;
    uint32_t acc = 0;
    for (size_t i = 0; i < n; i++) acc = lno32_add(acc, lno32_mul(x[i], x[i]));
    uint32_t mean = lno32_mul(acc, lno32_from_f32(1.0f / (float)n));
    uint32_t inv = lno32_recip(lno32_sqrt(lno32_add(mean, eps)));
    for (size_t i = 0; i < n; i++) dst[i] = lno32_mul(x[i], inv);
}

void lno32_softmax_row(const uint32_t *a, const uint32_t *mask, uint32_t *c, size_t n, uint32_t scale) {
    if (n == 0) return;
    uint32_t maxval = X32_NEG_INF;
    for (size_t i = 0; i < n; i++) {
        uint32_t v = a[i];
        if (v != X32_NEG_INF) {
            v = lno32_mul(v, scale);
            if (mask) {
                if (mask[i] == X32_NEG_INF) v = X32_NEG_INF;
                else if ((mask[i] & X32_LOGMASK) != 0) v = lno32_add(v, mask[i]);
            }
        }
        c[i] = v;
        if (lno32_gt(c[i], maxval)) maxval = c[i];
    }
    for (size_t i = 0; i < n; i++) c[i] = lno32_exp(lno32_sub(c[i], maxval));
    uint32_t total = c[0];
    for (size_t i = 1; i < n; i++) total = lno32_add(total, c[i]);
    for (size_t i = 0; i < n; i++) c[i] = lno32_div(c[i], total);
}

/* ======================================================================
 * Op drivers.
 * ==================================================================== */

/* lns_mul_mat (src/lns-ops.cpp:293-384): loops i13, i12, then every weight
 * row i0, then every activation row i1; one vec_dot per output. */
void lno16_mul_mat(int mode, const uint16_t *w, const float *x, float *dst,
                   int64_t K, int64_t M, int64_t N,
                   int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13) {
    const int64_t r2 = ne12 / ne02, r3 = ne13 / ne03;
    uint16_t *xb = (uint16_t *)malloc((size_t)(N * K > 0 ? N * K : 1) * sizeof(uint16_t));
    for (int64_t i13 = 0; i13 < ne13; i13++) {
        for (int64_t i12 = 0; i12 < ne12; i12++) {
            const float *xs = x + ((i13 * ne12 + i12) * N) * K;
            lno16_from_f32_n(xs, xb, (size_t)(N * K));
            const uint16_t *ws = w + (((i13 / r3) * ne02 + (i12 / r2)) * M) * K;
            float *ds = dst + ((i13 * ne12 + i12) * N) * M;
            for (int64_t m = 0; m < M; m++) {
                for (int64_t n = 0; n < N; n++) {
                    uint16_t d = lno16_vec_dot(mode, ws + m * K, xb + n * K, (size_t)K, &g_lfsr);
                    ds[n * M + m] = lno16_to_f32(d);
                }
            }
        }
    }
    free(xb);
}

void lno16_mul_mat_f32w(int mode, const float *w, const float *x, float *dst,
                        int64_t K, int64_t M, int64_t N,
                        int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13) {
    size_t nw = (size_t)(K * M * ne02 * ne03);
    uint16_t *wl = (uint16_t *)malloc((nw ? nw : 1) * sizeof(uint16_t));
    lno16_from_f32_n(w, wl, nw);
    lno16_mul_mat(mode, wl, x, dst, K, M, N, ne02, ne03, ne12, ne13);
    free(wl);
}

/* lns_mul_mat_id (src/lns-ops.cpp:394-462): for token t, slot s, expert
 * e = ids[t * neu + s], activation row i11 = s % ne11, each output row m in
 * turn (Monte draws in that order).  w: n_expert experts of M rows of K
 * xlns16 codes; x: [T][ne11][K] F32; dst: [T][neu][M] F32. */
void lno16_mul_mat_id(int mode, const uint16_t *w, const float *x, const int32_t *ids, float *dst,
                      int64_t K, int64_t M, int64_t n_expert, int64_t neu, int64_t T, int64_t ne11) {
    uint16_t *xb = (uint16_t *)malloc((size_t)(ne11 * K > 0 ? ne11 * K : 1) * sizeof(uint16_t));
    for (int64_t t = 0; t < T; t++) {
        lno16_from_f32_n(x + t * ne11 * K, xb, (size_t)(ne11 * K));
        for (int64_t s = 0; s < neu; s++) {
            const int32_t e = ids[t * neu + s];
            if (e < 0 || e >= n_expert) abort();   /* the reference's assert (:421) */
            const uint16_t *xr = xb + (s % ne11) * K;
            for (int64_t m = 0; m < M; m++) {
                uint16_t d = lno16_vec_dot(mode, w + (e * M + m) * K, xr, (size_t)K, &g_lfsr);
                dst[(t * neu + s) * M + m] = lno16_to_f32(d);
            }
        }
    }
    free(xb);
}

/* lns32_mul_mat_id (src32/lns32-ops.cpp:154-215), as lno16_mul_mat_id */
void lno32_mul_mat_id(const float *w, const float *x, const int32_t *ids, float *dst,
                      int64_t K, int64_t M, int64_t n_expert, int64_t neu, int64_t T, int64_t ne11) {
    size_t nw = (size_t)(K * M * n_expert);
    uint32_t *wl = (uint32_t *)malloc((nw ? nw : 1) * sizeof(uint32_t));
    uint32_t *xb = (uint32_t *)malloc((size_t)(ne11 * K > 0 ? ne11 * K : 1) * sizeof(uint32_t));
    lno32_from_f32_n(w, wl, nw);
    for (int64_t t = 0; t < T; t++) {
        lno32_from_f32_n(x + t * ne11 * K, xb, (size_t)(ne11 * K));
        for (int64_t s = 0; s < neu; s++) {
            const int32_t e = ids[t * neu + s];
            if (e < 0 || e >= n_expert) abort();
            const uint32_t *xr = xb + (s % ne11) * K;
            for (int64_t m = 0; m < M; m++)
                dst[(t * neu + s) * M + m] = lno32_to_f32(lno32_vec_dot(wl + (e * M + m) * K, xr, (size_t)K));
        }
    }
    free(wl);
    free(xb);
}

/* f32_mask_to_lns16 (src/lns-ops.cpp:634-637) */
static inline uint16_t mask16(float m) { return m <= -3.0e38f ? X16_NEG_INF : lno16_from_f32(m); }
static inline uint32_t mask32(float m) { return m <= -3.0e38f ? X32_NEG_INF : lno32_from_f32(m); }

/* lns_soft_max (src/lns-ops.cpp:643-695); mask row i1 of plane
 * (i2 % mne2, i3 % mne3) */
void lno16_soft_max(int mode, const float *src, const int64_t ne[4], const float *mask,
                    const int64_t mne[4], float scale, float *dst) {
    const int64_t n = ne[0];
    uint16_t *row = (uint16_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(uint16_t));
    uint16_t *mk = (uint16_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(uint16_t));
    const uint16_t sc = lno16_from_f32(scale);
    for (int64_t i3 = 0; i3 < ne[3]; i3++)
    for (int64_t i2 = 0; i2 < ne[2]; i2++)
    for (int64_t i1 = 0; i1 < ne[1]; i1++) {
        const int64_t r = (i3 * ne[2] + i2) * ne[1] + i1;
        lno16_from_f32_n(src + r * n, row, (size_t)n);
        if (mask) {
            const float *m = mask + (((i3 % mne[3]) * mne[2] + (i2 % mne[2])) * mne[1] + i1) * mne[0];
            for (int64_t i = 0; i < n; i++) mk[i] = mask16(m[i]);
        }
        lno16_softmax_row(mode, row, mask ? mk : NULL, row, (size_t)n, sc, &g_lfsr);
        lno16_to_f32_n(row, dst + r * n, (size_t)n);
    }
    free(row);
    free(mk);
}

/* lns_rms_norm (src/lns-ops.cpp:701-736) */
void lno16_rms_norm(int mode, const float *src, int64_t ncols, int64_t nrows, float eps, float *dst) {
    uint16_t *row = (uint16_t *)malloc((size_t)(ncols > 0 ? ncols : 1) * sizeof(uint16_t));
    const uint16_t e = lno16_from_f32(eps);
    for (int64_t r = 0; r < nrows; r++) {
        lno16_from_f32_n(src + r * ncols, row, (size_t)ncols);
        lno16_rms_norm_row(mode, row, row, (size_t)ncols, e, &g_lfsr);
        lno16_to_f32_n(row, dst + r * ncols, (size_t)ncols);
    }
    free(row);
}

/* lns32_mul_mat (src32/lns32-ops.cpp:98-144): weights converted from F32 */
void lno32_mul_mat_lnsw(const uint32_t *w, const float *x, float *dst,
                        int64_t K, int64_t M, int64_t N,
                        int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13) {
    const int64_t r2 = ne12 / ne02, r3 = ne13 / ne03;
    uint32_t *xb = (uint32_t *)malloc((size_t)(N * K > 0 ? N * K : 1) * sizeof(uint32_t));
    for (int64_t i13 = 0; i13 < ne13; i13++) {
        for (int64_t i12 = 0; i12 < ne12; i12++) {
            lno32_from_f32_n(x + ((i13 * ne12 + i12) * N) * K, xb, (size_t)(N * K));
            const uint32_t *ws = w + (((i13 / r3) * ne02 + (i12 / r2)) * M) * K;
            float *ds = dst + ((i13 * ne12 + i12) * N) * M;
            for (int64_t m = 0; m < M; m++)
                for (int64_t n = 0; n < N; n++)
                    ds[n * M + m] = lno32_to_f32(lno32_vec_dot(ws + m * K, xb + n * K, (size_t)K));
        }
    }
    free(xb);
}

void lno32_mul_mat(const float *w, const float *x, float *dst,
                   int64_t K, int64_t M, int64_t N,
                   int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13) {
    size_t nw = (size_t)(K * M * ne02 * ne03);
    uint32_t *wl = (uint32_t *)malloc((nw ? nw : 1) * sizeof(uint32_t));
    lno32_from_f32_n(w, wl, nw);
    lno32_mul_mat_lnsw(wl, x, dst, K, M, N, ne02, ne03, ne12, ne13);
    free(wl);
}

void lno32_soft_max(const float *src, const int64_t ne[4], const float *mask,
                    const int64_t mne[4], float scale, float *dst) {
    const int64_t n = ne[0];
    uint32_t *row = (uint32_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(uint32_t));
    uint32_t *mk = (uint32_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(uint32_t));
    const uint32_t sc = lno32_from_f32(scale);
    for (int64_t i3 = 0; i3 < ne[3]; i3++)
    for (int64_t i2 = 0; i2 < ne[2]; i2++)
    for (int64_t i1 = 0; i1 < ne[1]; i1++) {
        const int64_t r = (i3 * ne[2] + i2) * ne[1] + i1;
        lno32_from_f32_n(src + r * n, row, (size_t)n);
        if (mask) {
            const float *m = mask + (((i3 % mne[3]) * mne[2] + (i2 % mne[2])) * mne[1] + i1) * mne[0];
            for (int64_t i = 0; i < n; i++) mk[i] = mask32(m[i]);
        }
        lno32_softmax_row(row, mask ? mk : NULL, row, (size_t)n, sc);
        lno32_to_f32_n(row, dst + r * n, (size_t)n);
    }
    free(row);
    free(mk);
}

void lno32_rms_norm(const float *src, int64_t ncols, int64_t nrows, float eps, float *dst) {
    uint32_t *row = (uint32_t *)malloc((size_t)(ncols > 0 ? ncols : 1) * sizeof(uint32_t));
    const uint32_t e = lno32_from_f32(eps);
    for (int64_t r = 0; r < nrows; r++) {
        lno32_from_f32_n(src + r * ncols, row, (size_t)ncols);
        lno32_rms_norm_row(row, row, (size_t)ncols, e);
        lno32_to_f32_n(row, dst + r * ncols, (size_t)ncols);
    }
    free(row);
}

/* ======================================================================
 * Elementwise ops of the Llama graph (F32 in, F32 out, LNS inside).
 * ==================================================================== */

/* lns_add / lns_mul (src/lns-ops.cpp:468-530): b broadcast along rows
 * (b has nb elements, index i % nb) */
void lno16_add_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst) {
    for (int64_t i = 0; i < n; i++)
        dst[i] = lno16_to_f32(lno16_add(lno16_from_f32(a[i]), lno16_from_f32(b[i % nb])));
}
void lno16_mul_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst) {
    for (int64_t i = 0; i < n; i++)
        dst[i] = lno16_to_f32(lno16_mul(lno16_from_f32(a[i]), lno16_from_f32(b[i % nb])));
}

/* SCALE as the GPU backend computes it (cuda/lns-cuda-kernels.cuh:179-189):
 * y = x s, then + b when b != 0, with s and b converted once.  The CPU
 * backend's lns_scale (src/lns-ops.cpp:562-592) has the same arithmetic but
 * stores only into an LNS16 destination. */
void lno16_scale_f32(const float *src, int64_t n, float s, float b, float *dst) {
    const uint16_t sc = lno16_from_f32(s), bc = lno16_from_f32(b);
    for (int64_t i = 0; i < n; i++) {
        uint16_t v = lno16_mul(lno16_from_f32(src[i]), sc);
        if (b != 0.0f) v = lno16_add(v, bc);
        dst[i] = lno16_to_f32(v);
    }
}

/* lns_swiglu (src/lns-ops.cpp:812-868): silu(gate) * up */
void lno16_swiglu_f32(const float *gate, const float *up, int64_t n, float *dst) {
    for (int64_t i = 0; i < n; i++)
        dst[i] = lno16_to_f32(lno16_mul(lno16_silu(lno16_from_f32(gate[i])), lno16_from_f32(up[i])));
}

/* lns_rope (src/lns-ops.cpp:1199-1281), normal or NEOX pairs; x is
 * [ntok][nhead][ne0], pos[ntok]; cos/sin from the float recurrence
 * t *= theta_scale of the reference, theta_scale = powf(base, -2/n_dims) */
void lno16_rope_f32(const float *x, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                    int n_dims, int neox, float freq_base, float *dst) {
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    for (int64_t t = 0; t < ntok; t++)
    for (int64_t h = 0; h < nhead; h++) {
        const float *xr = x + (t * nhead + h) * ne0;
        float *yr = dst + (t * nhead + h) * ne0;
        float th = (float)pos[t];
        for (int64_t j = 0; j < n_dims; j += 2) {
            const uint16_t c = lno16_from_f32(cosf(th)), sn = lno16_from_f32(sinf(th));
            const int64_t i0 = neox ? j / 2 : j, i1 = neox ? j / 2 + n_dims / 2 : j + 1;
            const uint16_t x0 = lno16_from_f32(xr[i0]), x1 = lno16_from_f32(xr[i1]);
            yr[i0] = lno16_to_f32(lno16_sub(lno16_mul(x0, c), lno16_mul(x1, sn)));
            yr[i1] = lno16_to_f32(lno16_add(lno16_mul(x0, sn), lno16_mul(x1, c)));
            th *= theta_scale;
        }
        for (int64_t j = n_dims; j < ne0; j++) yr[j] = lno16_to_f32(lno16_from_f32(xr[j]));
    }
}

/* lns32_add / lns32_mul (src32/lns32-ops.cpp:224-282), b repeated every nb */
void lno32_add_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst) {
    for (int64_t i = 0; i < n; i++) dst[i] = lno32_to_f32(lno32_add(lno32_from_f32(a[i]), lno32_from_f32(b[i % nb])));
}
void lno32_mul_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst) {
    for (int64_t i = 0; i < n; i++) dst[i] = lno32_to_f32(lno32_mul(lno32_from_f32(a[i]), lno32_from_f32(b[i % nb])));
}

/* lns32_scale (src32/lns32-ops.cpp:318-342), as lno16_scale_f32 in xlns32 */
void lno32_scale_f32(const float *src, int64_t n, float s, float b, float *dst) {
    const uint32_t sc = lno32_from_f32(s), bc = lno32_from_f32(b);
    for (int64_t i = 0; i < n; i++) {
        uint32_t v = lno32_mul(lno32_from_f32(src[i]), sc);
        if (b != 0.0f) v = lno32_add(v, bc);
        dst[i] = lno32_to_f32(v);
    }
}

/* xlns32_silu (xlnscpp, absent): x times fp2xlns32 of the sigmoid of x's
 * value, the sigmoid formed in double and rounded to float.  Checked against
 * the eight swiglu values printed in unit-tests-lns32.txt (six decimals);
 * beyond those digits parity is unpinned. */
uint32_t lno32_silu(uint32_t x) {
    const double v = (double)lno32_to_f32(x);
    return lno32_mul(x, lno32_from_f32((float)(1.0 / (1.0 + exp(-v)))));
}

/* lns32_swiglu (src32/lns32-ops.cpp:535-587): silu(gate) * up */
void lno32_swiglu_f32(const float *gate, const float *up, int64_t n, float *dst) {
    for (int64_t i = 0; i < n; i++)
        dst[i] = lno32_to_f32(lno32_mul(lno32_silu(lno32_from_f32(gate[i])), lno32_from_f32(up[i])));
}

/* lns32_rope (src32/lns32-ops.cpp:795-880), normal or NEOX pairs; x is
 * [ntok][nhead][ne0], pos[ntok]; cos/sin from the same float recurrence as
 * the xlns16 rope; dims past n_dims round-trip through xlns32 */
void lno32_rope_f32(const float *x, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                    int n_dims, int neox, float freq_base, float *dst) {
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    for (int64_t t = 0; t < ntok; t++)
    for (int64_t h = 0; h < nhead; h++) {
        const float *xr = x + (t * nhead + h) * ne0;
        float *yr = dst + (t * nhead + h) * ne0;
        float th = (float)pos[t];
        for (int64_t j = 0; j < n_dims; j += 2) {
            const uint32_t c = lno32_from_f32(cosf(th)), sn = lno32_from_f32(sinf(th));
            const int64_t i0 = neox ? j / 2 : j, i1 = neox ? j / 2 + n_dims / 2 : j + 1;
            const uint32_t x0 = lno32_from_f32(xr[i0]), x1 = lno32_from_f32(xr[i1]);
            yr[i0] = lno32_to_f32(lno32_sub(lno32_mul(x0, c), lno32_mul(x1, sn)));
            yr[i1] = lno32_to_f32(lno32_add(lno32_mul(x0, sn), lno32_mul(x1, c)));
            th *= theta_scale;
        }
        for (int64_t j = n_dims; j < ne0; j++) yr[j] = lno32_to_f32(lno32_from_f32(xr[j]));
    }
}

/* ======================================================================
 * Table construction.
 * ==================================================================== */
/* xlns16_exp table: the direct (untabled) conversion of expf of the decoded
 * value.  Pinned by the ten printed softmax errors of
 * unit-tests-lns16-{base,sum32}.txt; the bucketed conversion table would
 * miss three of them. */
static uint16_t exp16_entry(uint16_t x) {
    return fp2xlns16_direct(expf(g_rev16[x]));
}

int lno_init(void) {
    if (g_ready) return 0;
    /* float -> xlns16: one entry per 2^15-wide bucket of float bit patterns,
     * the conversion of the bucket's lowest member */
    for (uint32_t i = 0; i < (1u << 17); i++) g_cvt16[i] = fp2xlns16_direct(f32_from_bits(i << 15));
    for (uint32_t i = 0; i < (1u << 16); i++) g_rev16[i] = rev16_entry((uint16_t)i);
    for (int d = 0; d <= X16_ESSZER; d++) {
        g_sb16[d] = sb16_entry(d);
        g_db16[d] = d == 0 ? 0 : db16_entry(d);
    }
    for (int d = X16_MC_START; d <= X16_MC_END; d++)
        g_mc16[d] = d < X16_MC_END ? (int32_t)floor(exp2(-(double)d / 128.0) * 185.0 * 64.0) : 0;
    for (uint32_t i = 0; i < (1u << 16); i++) g_exp16[i] = exp16_entry((uint16_t)i);
    for (uint32_t i = 0; i < (1u << 16); i++) {
        float v = g_rev16[i];
        g_sig16[i] = g_cvt16[bits_from_f32(1.0f / (1.0f + expf(-v))) >> 15];
    }

    for (int i = 0; i <= X32_SB_N; i++) g_sb32a[i] = (int32_t)truncl(sb32_exact((long double)i * (1 << X32_SB_SH)));
    for (int i = 0; i <= X32_SB_FN; i++)
        g_sb32b[i] = (int32_t)truncl(sb32_exact((long double)X32_SB_END + (long double)i * (1 << X32_SB_FSH)));
    g_db32a[0] = 0;
    for (int i = 1; i <= X32_DB_N; i++) g_db32a[i] = (int32_t)floorl(db32_exact((long double)i * (1 << X32_DB_SH)));
    for (int i = 0; i <= X32_DB_FN; i++)
        g_db32b[i] = (int32_t)floorl(db32_exact((long double)X32_DB_END + (long double)i * (1 << X32_DB_FSH)));
    for (size_t i = 0; i < sizeof g_sb32pm / sizeof g_sb32pm[0]; i++)
        g_sb32pm[i] = (int32_t)floorl(sb32_exact((long double)i * (1 << X32_PM_SH)));
    g_db32lo[0] = 0;
    for (int i = 1; i < (1 << X32_CO_SH); i++) g_db32lo[i] = (int32_t)floorl(db32_exact((long double)i));
    g_db32hi[0] = 0;
    for (int i = 1; i < (X32_CO_END >> X32_CO_SH); i++)
        g_db32hi[i] = (int32_t)floorl(db32_exact((long double)i * (1 << X32_CO_SH)));

    uint16_t s = 1;
    for (uint32_t i = 0; i < 65535u; i++) {
        g_lfsr_seq[i] = s;
        g_lfsr_log[s] = (uint16_t)i;
        s = lno_lfsr_step(s);
    }
    g_lfsr_log[0] = 0;
    g_lfsr = 7;
    g_ready = 1;
    return 0;
}
