/*
 * lns_oracle.h - CPU restatement of the reference's LNS16/LNS32 CPU backend.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * xlns-ggml-backend_amd/) links, loads or calls this code.  It is used by
 * tests/ as the parity checker, by __graft_entry__.smoke() as the checker of
 * one small GPU call, and by bench.py's cpu_baseline leg as the timed
 * single-threaded CPU reference.
 *
 * What it restates (paths relative to the reference checkout):
 *   - xlns16 / xlns32 arithmetic as configured by the reference build:
 *     xlnscpp xlns16.cpp with xlns16_table + xlns16_alt (src/CMakeLists.txt:13,
 *     src/lns-ops.cpp:40-53) and xlns32.cpp with xlns32_alt
 *     (src32/CMakeLists.txt:17).  xlnscpp itself is an absent submodule
 *     (pinned 41843b034689d5ca91e32a0043cc37265fb2ef5c,
 *     patches/xlnscpp-base-commit.txt:1); its published algorithm is restated
 *     here and pinned against the reference's committed outputs
 *     (the files of results/sum32-evidence/ and experiments/dot-product-scaling/results/
 *     convert.jsonl) by tests/test_oracle_pins.py.
 *   - the four xlns16 reductions (base, monte, lpvip, sum32):
 *     src/lns-ops.cpp:110-134, src/lns16-sum32.h, cuda/lns-cuda-xlns16.cu:67-130.
 *   - the op drivers lns_mul_mat (src/lns-ops.cpp:293-384), lns_soft_max
 *     (:643-695), lns_rms_norm (:701-736) and their xlns32 twins
 *     (src32/lns32-ops.cpp:98-144, 384-477), with the reference's loop and
 *     term order.
 *   - the process-global Monte LFSR and its reserve API (src/lns-ops.cpp:155-195).
 *
 * Parity status per function is listed in the header comment of
 * lns_oracle.c (pinned / partially pinned / parity unpinned).
 */
#ifndef LNS_ORACLE_H
#define LNS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* summation modes of the xlns16 reductions (GGML_LNS16_SUM) */
enum lno_mode { LNO_BASE = 0, LNO_MONTE = 1, LNO_LPVIP = 2, LNO_SUM32 = 3 };

int lno_init(void);

/* ---- xlns16 ---------------------------------------------------------- */
uint16_t lno16_from_f32(float x);
float    lno16_to_f32(uint16_t v);
void     lno16_from_f32_n(const float *src, uint16_t *dst, size_t n);
void     lno16_to_f32_n(const uint16_t *src, float *dst, size_t n);
uint16_t lno16_mul(uint16_t a, uint16_t b);
uint16_t lno16_div(uint16_t a, uint16_t b);
uint16_t lno16_add(uint16_t a, uint16_t b);
uint16_t lno16_sub(uint16_t a, uint16_t b);
uint16_t lno16_sqrt(uint16_t a);
uint16_t lno16_recip(uint16_t a);
uint16_t lno16_exp(uint16_t a);
uint16_t lno16_silu(uint16_t a);
int      lno16_gt(uint16_t a, uint16_t b);
/* exported tables (for tests): cvt[1<<17], sb/db[1281], exp[1<<16] */
const uint16_t *lno16_cvt_table(void);
const int16_t  *lno16_sb_table(void);
const int16_t  *lno16_db_table(void);
const uint16_t *lno16_exp_table(void);

/* widen / narrow of the sum32 and lpvip accumulators */
uint32_t lno16_widen(uint16_t v);
uint16_t lno16_narrow_sum32(uint32_t s);
uint16_t lno16_narrow_lpvip(uint32_t s);

/* reductions; lfsr is the Monte state (ignored by other modes) */
uint16_t lno16_sum(int mode, const uint16_t *a, size_t n, uint16_t *lfsr);
uint16_t lno16_vec_dot(int mode, const uint16_t *a, const uint16_t *b, size_t n, uint16_t *lfsr);
void     lno16_rms_norm_row(int mode, const uint16_t *x, uint16_t *dst, size_t n, uint16_t eps, uint16_t *lfsr);
void     lno16_softmax_row(int mode, const uint16_t *a, const uint16_t *mask, uint16_t *c, size_t n,
                           uint16_t scale, uint16_t *lfsr);
uint16_t lno16_add_monte(uint16_t a, uint16_t b, uint16_t *lfsr);
/* Monte dither threshold F(d) for d0 .. d0 + n - 1 (0 outside [1091, 1732)) */
void lno16_monte_threshold_n(int d0, int n, int32_t *out);
uint32_t lno16_lpvip_add(uint32_t acc, uint16_t t);
void     lno32_lpvip_db_n(uint32_t d0, uint32_t n, int32_t *out);

/* ---- Monte LFSR (process-global, seed 7) ------------------------------ */
uint16_t lno_lfsr_step(uint16_t s);
uint16_t lno_lfsr_jump(uint16_t s, uint64_t n);
int      lno_monte_get_state(uint16_t *state);
int      lno_monte_set_state(uint16_t state);
int      lno_monte_reserve(uint64_t draws, uint16_t *start);

/* ---- xlns32 ---------------------------------------------------------- */
uint32_t lno32_from_f32(float x);
float    lno32_to_f32(uint32_t v);
void     lno32_from_f32_n(const float *src, uint32_t *dst, size_t n);
void     lno32_to_f32_n(const uint32_t *src, float *dst, size_t n);
uint32_t lno32_mul(uint32_t a, uint32_t b);
uint32_t lno32_div(uint32_t a, uint32_t b);
uint32_t lno32_add(uint32_t a, uint32_t b);
uint32_t lno32_sub(uint32_t a, uint32_t b);
uint32_t lno32_sqrt(uint32_t a);
uint32_t lno32_recip(uint32_t a);
uint32_t lno32_exp(uint32_t a);
int      lno32_gt(uint32_t a, uint32_t b);
const int32_t *lno32_table(const char *name, size_t *n);
/* 0: the restated xlns32_alt adder (default); 1: its sb replaced by the one
 * the reference's experiments ran with (tests only); returns the old value */
int      lno32_set_variant(int v);
uint32_t lno32_vec_dot(const uint32_t *a, const uint32_t *b, size_t n);
void     lno32_rms_norm_row(const uint32_t *x, uint32_t *dst, size_t n, uint32_t eps);
void     lno32_softmax_row(const uint32_t *a, const uint32_t *mask, uint32_t *c, size_t n, uint32_t scale);

/* ---- op drivers (ggml semantics; contiguous tensors, ne[0] fastest) ---- */
/* dst[i13][i12][n][m] = sum_k w[(i13/r3)][(i12/r2)][m][k] * x[i13][i12][n][k]
 * w: xlns16 codes [ne03][ne02][M][K]; x: F32 [ne13][ne12][N][K]; dst: F32 */
void lno16_mul_mat(int mode, const uint16_t *w, const float *x, float *dst,
                   int64_t K, int64_t M, int64_t N,
                   int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13);
void lno16_mul_mat_id(int mode, const uint16_t *w, const float *x, const int32_t *ids, float *dst,
                      int64_t K, int64_t M, int64_t n_expert, int64_t neu, int64_t T, int64_t ne11);
void lno32_mul_mat_id(const float *w, const float *x, const int32_t *ids, float *dst,
                      int64_t K, int64_t M, int64_t n_expert, int64_t neu, int64_t T, int64_t ne11);
void lno16_mul_mat_f32w(int mode, const float *w, const float *x, float *dst,
                        int64_t K, int64_t M, int64_t N,
                        int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13);
/* src F32 [ne3][ne2][ne1][ne0]; mask (optional) F32 [mne3][mne2][mne1>=ne1][ne0] */
void lno16_soft_max(int mode, const float *src, const int64_t ne[4], const float *mask,
                    const int64_t mne[4], float scale, float *dst);
void lno16_rms_norm(int mode, const float *src, int64_t ncols, int64_t nrows, float eps, float *dst);

void lno16_add_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst);
void lno16_mul_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst);
void lno16_scale_f32(const float *src, int64_t n, float s, float b, float *dst);
void lno16_swiglu_f32(const float *gate, const float *up, int64_t n, float *dst);
void lno16_rope_f32(const float *x, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                    int n_dims, int neox, float freq_base, float *dst);

void lno32_mul_mat(const float *w, const float *x, float *dst,
                   int64_t K, int64_t M, int64_t N,
                   int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13);
void lno32_mul_mat_lnsw(const uint32_t *w, const float *x, float *dst,
                        int64_t K, int64_t M, int64_t N,
                        int64_t ne02, int64_t ne03, int64_t ne12, int64_t ne13);
void lno32_soft_max(const float *src, const int64_t ne[4], const float *mask,
                    const int64_t mne[4], float scale, float *dst);
void lno32_rms_norm(const float *src, int64_t ncols, int64_t nrows, float eps, float *dst);
uint32_t lno32_silu(uint32_t x);
void lno32_add_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst);
void lno32_mul_f32(const float *a, const float *b, int64_t n, int64_t nb, float *dst);
void lno32_scale_f32(const float *src, int64_t n, float s, float b, float *dst);
void lno32_swiglu_f32(const float *gate, const float *up, int64_t n, float *dst);
void lno32_rope_f32(const float *x, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                    int n_dims, int neox, float freq_base, float *dst);

#ifdef __cplusplus
}
#endif

#endif
