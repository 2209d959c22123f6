// Host construction of the xlns16 / xlns32 arithmetic tables.
//
// The formulas are xlnscpp's (pinned 41843b0, patches/xlnscpp-base-commit.txt)
// as the reference configures it: xlns16_table + xlns16_alt for xlns16
// (lns-backend/src/CMakeLists.txt:13) and xlns32_alt for xlns32
// (src32/CMakeLists.txt:17).
#include "lnship_tables.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace lnship {
namespace {

float bits_to_float(uint32_t b) {
    float f;
    std::memcpy(&f, &b, sizeof f);
    return f;
}

// (int16_t)(double) as x86-64 code computes it: truncation to a 32-bit
// integer (0x80000000 when out of range or NaN), then the low 16 bits.
int16_t to_s16(double v) {
    int32_t i = (v > -2147483649.0 && v < 2147483648.0) ? (int32_t)v : INT32_MIN;
    return (int16_t)(uint16_t)(uint32_t)i;
}
int32_t to_s32(double v) {
    return (v > -2147483649.0 && v < 2147483648.0) ? (int32_t)v : INT32_MIN;
}

// float -> xlns16 without the table: log truncated toward zero, offset by
// xor with 0x4000.
uint16_t encode16(float x) {
    if (x == 0.0f) return 0;
    if (x > 0.0f) {
        uint16_t l = (uint16_t)to_s16((std::log((double)x) / std::log(2.0)) * 128.0);
        return (uint16_t)((l & k16_logmask) ^ k16_one);
    }
    uint16_t l = (uint16_t)to_s16((std::log(std::fabs((double)x)) / std::log(2.0)) * 128.0);
    return (uint16_t)((l | k16_sign) ^ k16_one);
}

float decode16_exact(uint16_t v) {
    if ((v & k16_logmask) == 0) return 0.0f;
    double m = std::pow(2.0, (double)(int16_t)(uint16_t)((v & k16_logmask) - k16_one) / 128.0);
    return (float)((v & k16_sign) ? -m : m);
}

// The decode table stores each value as a 7-significant-digit decimal.
float decode16_table(uint16_t v) {
    float f = decode16_exact(v);
    if (f == 0.0f) return f;
    char buf[48];
    std::snprintf(buf, sizeof buf, "%e", (double)f);
    return (float)std::strtod(buf, nullptr);
}

long double gauss32_sb(long double d) { return log2l(1.0L + exp2l(-d / 8388608.0L)) * 8388608.0L; }
long double gauss32_db(long double d) { return log2l(1.0L - exp2l(-d / 8388608.0L)) * 8388608.0L; }

}  // namespace

void build_host_tables(host_tables &t) {
    for (uint32_t i = 0; i < (1u << 17); i++) t.cvt16[i] = encode16(bits_to_float(i << 15));
    for (uint32_t i = 0; i < (1u << 16); i++) t.rev16[i] = decode16_table((uint16_t)i);

    // xlns16_alt adjust at distance d: -d + (int)(log2(+-1 + 2^(d/128))*128 + .5)
    for (int d = 0; d < k16_gauss_n; d++) {
        int16_t sb = 0, db = 0;
        if (d <= k16_esszer) {
            double vs = std::log(1.0 + std::pow(2.0, (double)d / 128.0)) / std::log(2.0) * 128.0 + 0.5;
            sb = (int16_t)(-d + to_s32(vs));
            if (d > 0) {
                double vd = std::log(-1.0 + std::pow(2.0, (double)d / 128.0)) / std::log(2.0) * 128.0 + 0.5;
                db = (int16_t)(-d + to_s32(vd));
            }
        }
        t.gauss16[d] = sb;
        t.gauss16[k16_gauss_n + d] = db;
    }
    // Monte (layout in lnship_tables.h); db at distance 0 is left to the
    // caller (exact cancellation)
    for (int d = 0; d < k16_mc_n; d++) {
        int32_t *e = t.gauss16m + 4 * d;
        if (d < k16_mc_start) {
            e[0] = (int32_t)t.gauss16[d] * 64;
            e[1] = 0;
            e[2] = (int32_t)t.gauss16[k16_gauss_n + d] * 64;
            e[3] = 0;
        } else {
            const int32_t f = d < k16_mc_end ? (int32_t)std::floor(std::exp2(-(double)d / 128.0) * 185.0 * 64.0) : 0;
            e[0] = f;
            e[1] = 63;
            e[2] = 64 - f;
            e[3] = -1;
        }
    }

    for (uint32_t i = 0; i < (1u << 16); i++) t.exp16[i] = encode16(std::exp(t.rev16[i]));
    // the sigmoid goes through the bucketed conversion table
    for (uint32_t i = 0; i < (1u << 16); i++) {
        float sg = 1.0f / (1.0f + std::exp(-t.rev16[i]));
        uint32_t b;
        std::memcpy(&b, &sg, sizeof b);
        t.sig16[i] = t.cvt16[b >> 15];
    }

    int32_t *p = t.tab32;
    for (int i = 0; i < k32_sb_n; i++)
        p[k32_off_sb + i] = (int32_t)truncl(gauss32_sb((long double)i * (1 << k32_sb_sh)));
    for (int i = 0; i < k32_sb_fn; i++)
        p[k32_off_sbf + i] = (int32_t)truncl(gauss32_sb((long double)k32_sb_end + (long double)i * (1 << k32_sb_fsh)));
    for (int i = 0; i < k32_db_n; i++)
        p[k32_off_db + i] = (int32_t)floorl(gauss32_db((long double)(i + k32_db_first) * (1 << k32_db_sh)));
    for (int i = 0; i < k32_db_fn; i++)
        p[k32_off_dbf + i] = (int32_t)floorl(gauss32_db((long double)k32_db_end + (long double)i * (1 << k32_db_fsh)));
    p[k32_off_dlo] = 0;
    for (int i = 1; i < k32_co_n; i++) p[k32_off_dlo + i] = (int32_t)floorl(gauss32_db((long double)i));
    p[k32_off_dhi] = 0;
    for (int i = 1; i < k32_co_n; i++)
        p[k32_off_dhi + i] = (int32_t)floorl(gauss32_db((long double)i * (1 << k32_co_sh)));

    uint16_t s = 1;
    for (uint32_t i = 0; i < 65535u; i++) {
        t.lfsr_seq[i] = s;
        t.lfsr_log[s] = (uint16_t)i;
        uint16_t bit = s & 1u;
        s >>= 1;
        if (bit) s ^= 0xB400u;
    }
    t.lfsr_seq[65535] = t.lfsr_seq[0];
    t.lfsr_log[0] = 0;
    for (int k = 0; k < k_lp_n; k++) {
        t.lpdb[k] = std::exp2(-(double)k / 256.0);
        t.lpdb[k_lp_n + k] = 1.0 / (1.0 + (double)k / 256.0);
        t.lpdb[2 * k_lp_n + k] = std::log2(1.0 + (double)k / 256.0);
    }
}

}  // namespace lnship
