// Device-side xlns16 / xlns32 arithmetic for gfx950.
//
// Bit-for-bit the operations of the reference CPU backend (xlnscpp with
// xlns16_table + xlns16_alt, xlns32_alt; see lnship_tables.cpp), written as
// branch-light integer code: a wave runs 64 independent reductions, one per
// lane, and every reduction keeps the reference's term order.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "lnship_tables.h"

namespace lnship {

// Device copies of the tables (global memory; the hot ones are staged in LDS
// by the kernels that need them).
struct dev_tables {
    const uint16_t *cvt16;
    const float *rev16;
    const int16_t *gauss16;
    const int32_t *gauss16m;   // the Monte adder's LDS image (host_tables::gauss16m, db's dither entries as (-F, 63))
    const uint16_t *exp16;
    const uint16_t *sig16;
    const int32_t *tab32;
    const int32_t *lds32;   // the LDS image of the xlns32 adder tables (after the descriptors)
    const int32_t *lds32d;  // the same as the single-chain step reads it (dhi pairs' first words as ksb - th2)
    const int32_t *pos32;   // the LDS image of the positive-sum adder (sb's (node, scaled slope) pairs)
    const uint16_t *lfsr_seq;
    const uint16_t *lfsr_log;
    const uint16_t *rho16;  // rho16[c] = cvt16 of rev16[c]: a code through F32 and back, as between graph nodes
    const double *lpdb;     // lpvip's db tables (host_tables::lpdb)
};

__device__ __forceinline__ uint32_t f32_bits(float f) { return __float_as_uint(f); }

// ---- xlns16 ------------------------------------------------------------

__device__ __forceinline__ uint32_t x16_from_f32(const uint16_t *cvt, float f) { return cvt[f32_bits(f) >> 15]; }

// xlns16_mul: log fields added, clamped to [0, 0x7fff] (underflow gives a
// signed zero, overflow saturates), sign xor.
__device__ __forceinline__ uint32_t x16_mul(uint32_t x, uint32_t y) {
    int32_t l = (int32_t)(x & k16_logmask) + (int32_t)(y & k16_logmask) - (int32_t)k16_one;
    l = min(max(l, 0), (int32_t)k16_logmask);
    return ((x ^ y) & k16_sign) | (uint32_t)l;
}

__device__ __forceinline__ uint32_t x16_div(uint32_t x, uint32_t y) {
    int32_t l = (int32_t)(x & k16_logmask) - (int32_t)(y & k16_logmask) + (int32_t)k16_one;
    l = min(max(l, 0), (int32_t)k16_logmask);
    return ((x ^ y) & k16_sign) | (uint32_t)l;
}

__device__ __forceinline__ uint32_t x16_recip(uint32_t x) {
    return (x & k16_sign) | ((0u - x) & k16_logmask);
}

// log field halved, rounding half away from zero, sign dropped
__device__ __forceinline__ uint32_t x16_sqrt(uint32_t x) {
    int32_t sh = (int32_t)(int16_t)(uint16_t)(x << 1);
    int32_t q = sh / 4;
    return ((uint32_t)q & k16_logmask) ^ 0x2000u;
}

__device__ __forceinline__ int32_t x16_canon(uint32_t x) {
    return (int32_t)(int16_t)(uint16_t)((x & k16_sign) ? (x ^ k16_logmask) : x);
}

// xlns16_add (xlns16_alt): the larger operand times 2^(adj/128), adj from
// the Gaussian-log table at distance d (g: sb at [0..], db at [k16_gauss_n..];
// entries past the essential zero are 0).
__device__ __forceinline__ uint32_t x16_add_g(const int16_t *g, uint32_t x, uint32_t y) {
    uint32_t xl = x & k16_logmask, yl = y & k16_logmask;
    uint32_t maxl = max(xl, yl), d = maxl - min(xl, yl);
    uint32_t sgn = (xl > yl ? x : y) & k16_sign;
    uint32_t usedb = (x ^ y) & k16_sign;
    int32_t adj = g[min(d, (uint32_t)k16_esszer + 1) + (usedb ? k16_gauss_n : 0)];
    int32_t l = min(max((int32_t)maxl + adj, 0), (int32_t)k16_logmask);
    uint32_t r = sgn | (uint32_t)l;
    return (d == 0 && usedb) ? 0u : r;
}

// The Monte LFSR: one step per Monte addition (Galois, taps 0xB400).
__device__ __forceinline__ uint32_t lfsr_step(uint32_t s) {
    return (s >> 1) ^ ((s & 1u) ? 0xB400u : 0u);
}

// ---- xlns32 ------------------------------------------------------------

// Linear interpolation between grid nodes t[i], t[i+1], floored.
__device__ __forceinline__ int32_t interp32(const int32_t *t, uint32_t i, uint32_t f, int sh) {
    int32_t t0 = t[i], t1 = t[i + 1];
    return t0 + (int32_t)((int64_t)(t1 - t0) * (int64_t)f >> sh);
}

__device__ __forceinline__ int32_t sb32(const int32_t *T, uint32_t d) {   // d < esszer
    if (d < k32_sb_end) return interp32(T + k32_off_sb, d >> k32_sb_sh, d & ((1u << k32_sb_sh) - 1), k32_sb_sh);
    uint32_t e = d - k32_sb_end;
    return interp32(T + k32_off_sbf, e >> k32_sb_fsh, e & ((1u << k32_sb_fsh) - 1), k32_sb_fsh);
}

__device__ __forceinline__ int32_t db32(const int32_t *T, uint32_t d) {   // 0 < d < esszer
    if (d >= k32_co_end) {
        if (d < k32_db_end)
            return interp32(T + k32_off_db, (d >> k32_db_sh) - k32_db_first, d & ((1u << k32_db_sh) - 1), k32_db_sh);
        uint32_t e = d - k32_db_end;
        return interp32(T + k32_off_dbf, e >> k32_db_fsh, e & ((1u << k32_db_fsh) - 1), k32_db_fsh);
    }
    // cotransformation: 1 - 2^-d = (1 - 2^-dh) + 2^-dh (1 - 2^-dl)
    uint32_t dl = d & ((1u << k32_co_sh) - 1), dh = d - dl;
    int32_t lo = T[k32_off_dlo + dl];
    if (dh == 0) return lo;
    int32_t th = T[k32_off_dhi + (dh >> k32_co_sh)];
    if (dl == 0) return th;
    uint32_t e = (uint32_t)((int32_t)dh - lo + th);
    return th + (e < k32_esszer ? sb32(T, e) : 0);
}

// xlns32_add (xlns32_alt), same structure as the xlns16 adder
__device__ __forceinline__ uint32_t x32_add(const int32_t *T, uint32_t x, uint32_t y) {
    uint32_t xl = x & k32_logmask, yl = y & k32_logmask;
    uint32_t maxl = max(xl, yl), d = maxl - min(xl, yl);
    uint32_t sgn = (xl > yl ? x : y) & k32_sign;
    uint32_t usedb = (x ^ y) & k32_sign;
    if (d == 0 && usedb) return 0u;
    int32_t adj = 0;
    if (d < k32_esszer) adj = usedb ? db32(T, d) : sb32(T, d);
    // xlns32_mul(maxxy, 0x40000000 + adj): underflow -> signed zero,
    // overflow -> saturation
    uint32_t s = maxl + (uint32_t)adj;
    uint32_t l = (s & k32_sign) ? ((s & k32_one) ? 0u : k32_logmask) : s;
    return sgn | l;
}

// The product's log is the sum of the logs less the offset, clamped to the
// field: an underflow gives log 0 (zero), an overflow the largest log.  The
// sum of two 31-bit logs fits 32 bits, so one unsigned median does both
// clamps before the offset comes off.
__device__ __forceinline__ uint32_t x32_mul(uint32_t x, uint32_t y) {
    const uint32_t l = min(max((x & k32_logmask) + (y & k32_logmask), k32_one), k32_one + k32_logmask);
    return ((x ^ y) & k32_sign) | (l - k32_one);
}

__device__ __forceinline__ uint32_t x32_div(uint32_t x, uint32_t y) {
    uint32_t t = (x & k32_logmask) - (y & k32_logmask) + k32_one;
    uint32_t s = (x ^ y) & k32_sign;
    if (t & k32_sign) return (t & k32_one) ? s : (s | k32_logmask);
    return s | t;
}

__device__ __forceinline__ uint32_t x32_recip(uint32_t x) { return (x & k32_sign) | ((0u - x) & k32_logmask); }

__device__ __forceinline__ uint32_t x32_sqrt(uint32_t x) {
    int32_t sh = (int32_t)(x << 1);
    int32_t q = sh / 4;
    return ((uint32_t)q & k32_logmask) ^ 0x20000000u;
}

__device__ __forceinline__ int32_t x32_canon(uint32_t x) {
    return (int32_t)((x & k32_sign) ? (x ^ k32_logmask) : x);
}

// float -> xlns32: 2^23*log2|x| truncated toward zero.  The binade's
// fraction log2(1.m) is evaluated in double: its error (< 2^-29 units) only
// matters within that distance of an integer, which no mantissa comes near.
__device__ __forceinline__ uint32_t x32_from_f32(float f) {
    uint32_t b = f32_bits(f);
    uint32_t s = b & 0x80000000u;
    uint32_t ex = (b >> 23) & 0xffu, mt = b & 0x7fffffu;
    if (ex == 0 && mt == 0) return 0u;
    if (ex == 0xffu) return mt ? (0x80000000u ^ k32_one) : (s ? (0x80000000u ^ k32_one) : k32_one);
    int64_t l;
    if (ex == 0) {
        // denormal: log2(m) - 149
        double lg = log2((double)mt) - 149.0;
        double v = lg * 8388608.0;
        l = (int64_t)v;   // toward zero
    } else {
        int32_t e = (int32_t)ex - 127;
        double fr = log2(1.0 + (double)mt * (1.0 / 8388608.0)) * 8388608.0;  // [0, 2^23)
        int64_t fl = (int64_t)fr;                       // floor (fr >= 0)
        bool exact = (double)fl == fr;
        if (e >= 0) l = (int64_t)e * 8388608 + fl;
        else l = (int64_t)e * 8388608 + fl + (exact ? 0 : 1);   // toward zero
    }
    uint32_t li = (uint32_t)(int32_t)l;
    if (!s) return (li & k32_logmask) ^ k32_one;
    return (li | k32_sign) ^ k32_one;
}

// xlns32 -> float, correctly rounded 2^(L/2^23)
__device__ __forceinline__ float x32_to_f32(uint32_t v) {
    if ((v & k32_logmask) == 0) return 0.0f;
    int32_t l = (int32_t)((v & k32_logmask) - k32_one);
    int32_t q = l >> 23;                  // floor
    int32_t r = l - q * 8388608;          // [0, 2^23)
    double m = exp2((double)r * (1.0 / 8388608.0));
    float f = (float)ldexp(m, q);
    return (v & k32_sign) ? -f : f;
}

}  // namespace lnship
