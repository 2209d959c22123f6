/*
 * ggml_host.c - TEST INFRASTRUCTURE: a stand-in for the ggml-base functions
 * the LNSHIP ggml backends import (the list in
 * xlns-ggml-backend_amd/csrc/ggml_abi.h), so tests can load
 * libggml-lnship.so and drive it through its registry / device / backend
 * vtables without a ggml build.  Its op and type numbering is its own: the
 * backend matches ops and types by name only.
 */
#include "ggml_abi.h"

#include <stdlib.h>
#include <string.h>

/* ---- ops -------------------------------------------------------------- */
static const char *const k_ops[] = {"NONE", "DUP", "ADD", "MUL", "DIV", "SCALE", "RMS_NORM", "MUL_MAT", "SOFT_MAX",
                                    "ROPE", "GLU", "UNARY", "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS",
                                    "CPY", "CONT", "SET_ROWS", "MUL_MAT_ID"};
static const char *const k_glu[] = {"REGLU", "GEGLU", "SWIGLU"};
static const char *const k_unary[] = {"ABS", "NEG", "TANH", "RELU", "GELU", "SILU"};
#define N_OPS ((int)(sizeof k_ops / sizeof k_ops[0]))

int ggml_host_op(const char *name) {
    for (int i = 0; i < N_OPS; i++)
        if (!strcmp(k_ops[i], name)) return i;
    return -1;
}
int ggml_host_glu(const char *name) {
    for (int i = 0; i < 3; i++)
        if (!strcmp(k_glu[i], name)) return i;
    return -1;
}
int ggml_host_unary(const char *name) {
    for (int i = 0; i < 6; i++)
        if (!strcmp(k_unary[i], name)) return i;
    return -1;
}

const char *ggml_op_name(enum ggml_op op) { return (int)op >= 0 && (int)op < N_OPS ? k_ops[op] : "UNKNOWN"; }

const char *ggml_op_desc(const struct ggml_tensor *t) {
    const int op = (int)t->op;
    if (op == ggml_host_op("GLU") && t->op_params[0] >= 0 && t->op_params[0] < 3) return k_glu[t->op_params[0]];
    if (op == ggml_host_op("UNARY") && t->op_params[0] >= 0 && t->op_params[0] < 6) return k_unary[t->op_params[0]];
    return ggml_op_name(t->op);
}

/* ---- types: f32, f16, q8_0 (block of 32 int8 + half scale), q4_K, i32, i64, lns16 --- */
static float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal: renormalise */
            uint32_t mm = m, ee = 113;
            while (!(mm & 0x400)) {
                mm <<= 1;
                ee--;
            }
            bits = s | (ee << 23) | ((mm & 0x3ff) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void f16_to_float(const void *x, float *y, int64_t k) {
    const uint16_t *h = (const uint16_t *)x;
    for (int64_t i = 0; i < k; i++) y[i] = half_to_float(h[i]);
}

static void q8_0_to_float(const void *x, float *y, int64_t k) {
    const uint8_t *b = (const uint8_t *)x;
    for (int64_t i = 0; i < k / 32; i++, b += 34) {
        uint16_t dh;
        memcpy(&dh, b, 2);
        const float d = half_to_float(dh);
        for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
    }
}

/* Q4_K, ggml's published block of 256 (144 bytes): half d, half dmin,
 * 12 bytes of eight 6-bit (scale, min) pairs, 128 bytes of 4-bit quants.
 * Sub-block j (32 values) has scale sc_j and min m_j: pairs 0-3 are the low
 * 6 bits of bytes j and j + 4; pairs 4-7 take their low 4 bits from byte
 * j + 4 (scale: low nibble, min: high nibble) and their top 2 bits from the
 * top 2 bits of bytes j - 4 (scale) and j (min).  Quants come in 32-byte
 * runs: the low nibbles of a run are sub-block 2i, its high nibbles 2i + 1;
 * value = d * sc * q - dmin * m. */
static void q4_k_pair(int j, const uint8_t *s, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void q4_k_to_float(const void *x, float *y, int64_t k) {
    const uint8_t *b = (const uint8_t *)x;
    for (int64_t i = 0; i < k / 256; i++, b += 144) {
        uint16_t dh, mh;
        memcpy(&dh, b, 2);
        memcpy(&mh, b + 2, 2);
        const float d = half_to_float(dh), dmin = half_to_float(mh);
        const uint8_t *sc = b + 4, *q = b + 16;
        for (int r = 0; r < 4; r++, q += 32) {
            int s0, m0, s1, m1;
            q4_k_pair(2 * r, sc, &s0, &m0);
            q4_k_pair(2 * r + 1, sc, &s1, &m1);
            const float d0 = d * (float)s0, o0 = dmin * (float)m0, d1 = d * (float)s1, o1 = dmin * (float)m1;
            for (int l = 0; l < 32; l++) *y++ = d0 * (float)(q[l] & 15) - o0;
            for (int l = 0; l < 32; l++) *y++ = d1 * (float)(q[l] >> 4) - o1;
        }
    }
}

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_I32 = 26, T_I64 = 27, T_LNS16 = 43, T_COUNT = 44 };

static struct ggml_type_traits k_traits[T_COUNT];

static void init_traits(void) {
    static int done = 0;
    if (done) return;
    done = 1;
    for (int i = 0; i < T_COUNT; i++) k_traits[i].type_name = "unused";
    k_traits[T_F32] = (struct ggml_type_traits){"f32", 1, 0, 4, false, NULL, NULL};
    k_traits[T_F16] = (struct ggml_type_traits){"f16", 1, 0, 2, false, f16_to_float, NULL};
    k_traits[T_Q8_0] = (struct ggml_type_traits){"q8_0", 32, 0, 34, true, q8_0_to_float, NULL};
    k_traits[T_Q4_K] = (struct ggml_type_traits){"q4_K", 256, 0, 144, true, q4_k_to_float, NULL};
    k_traits[T_I32] = (struct ggml_type_traits){"i32", 1, 0, 4, false, NULL, NULL};
    k_traits[T_I64] = (struct ggml_type_traits){"i64", 1, 0, 8, false, NULL, NULL};
    k_traits[T_LNS16] = (struct ggml_type_traits){"lns16", 1, 0, 2, false, NULL, NULL};
}

const struct ggml_type_traits *ggml_get_type_traits(enum ggml_type t) {
    init_traits();
    return &k_traits[(int)t];
}
const char *ggml_type_name(enum ggml_type t) { return ggml_get_type_traits(t)->type_name; }
size_t ggml_type_size(enum ggml_type t) { return ggml_get_type_traits(t)->type_size; }
int64_t ggml_blck_size(enum ggml_type t) { return ggml_get_type_traits(t)->blck_size; }

/* ---- buffers (the layouts of ggml_abi.h) ------------------------------ */
static struct ggml_backend_buffer_type k_cpu_buft; /* iface unused: is_host answers by identity */

ggml_backend_buffer_type_t ggml_backend_cpu_buffer_type(void) { return &k_cpu_buft; }
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t b) { return b == &k_cpu_buft; }

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void *context, size_t size) {
    struct ggml_backend_buffer *b = (struct ggml_backend_buffer *)calloc(1, sizeof *b);
    b->iface = iface;
    b->buft = buft;
    b->context = context;
    b->size = size;
    b->usage = GGML_BACKEND_BUFFER_USAGE_ANY;
    return b;
}

ggml_backend_buffer_t ggml_backend_cpu_buffer_from_ptr(void *ptr, size_t size) {
    struct ggml_backend_buffer_i none;
    memset(&none, 0, sizeof none);
    (void)ptr;
    return ggml_backend_buffer_init(&k_cpu_buft, none, NULL, size);
}

enum ggml_backend_buffer_usage ggml_backend_buffer_get_usage(ggml_backend_buffer_t b) { return b->usage; }
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t b) { return b->buft; }

/* ggml.c's ggml_nbytes */
size_t ggml_nbytes(const struct ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] <= 0) return 0;
    const size_t blck = (size_t)ggml_blck_size(t->type);
    size_t n = blck == 1 ? ggml_type_size(t->type) : (size_t)t->ne[0] * t->nb[0] / blck;
    for (int i = blck == 1 ? 0 : 1; i < GGML_MAX_DIMS; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    return n;
}

/* a host buffer handle with the given usage (0 any, 1 weights, 2 compute) */
ggml_backend_buffer_t ggml_host_buffer(int usage) {
    ggml_backend_buffer_t b = ggml_backend_cpu_buffer_from_ptr(NULL, 0);
    b->usage = (enum ggml_backend_buffer_usage)usage;
    return b;
}

/* set a buffer's usage (ggml_backend_buffer_set_usage) */
void ggml_host_set_usage(ggml_backend_buffer_t b, int usage) { b->usage = (enum ggml_backend_buffer_usage)usage; }

size_t ggml_host_sizeof_tensor(void) { return sizeof(struct ggml_tensor); }
size_t ggml_host_offsetof_data(void) { return offsetof(struct ggml_tensor, data); }
size_t ggml_host_offsetof_name(void) { return offsetof(struct ggml_tensor, name); }
size_t ggml_host_offsetof_src(void) { return offsetof(struct ggml_tensor, src); }
