/*
 * ggml-lnship.h - the lnship library as ggml backends.
 *
 * LNS arithmetic on an AMD Instinct GPU (gfx950) through hand-written HIP
 * kernels.  Two devices, like the reference's LNSCUDA backend
 * (lns-backend/include/ggml-lns-cuda.h:10-23):
 *   LNSHIP16 - xlns16 in the summation mode GGML_LNS16_SUM names (base,
 *              monte, lpvip or sum32), read at run time (default base).
 *              Every mode is bit-exact against the repository's CPU
 *              restatement of the LNS16 backend (oracle/).  Against the
 *              reference's own printed outputs: base reproduces every one;
 *              sum32 every one except two figures of its xlns32_alt adder;
 *              monte 13 of its 15 unit-test figures (its xlnscpp source is
 *              absent; the restated dither is fitted to the printed
 *              figures); lpvip none (its source is absent too).
 *   LNSHIP32 - xlns32, bit-exact against the restated LNS32 backend, whose
 *              xlns32_alt adder misses two of the reference's printed
 *              LNS32 figures.
 * Both are ACCEL devices on host buffers: ggml keeps every tensor in host
 * memory, each op uploads its inputs and downloads its result, and weights
 * (tensors in GGML_BACKEND_BUFFER_USAGE_WEIGHTS buffers) are converted to LNS
 * once and kept in HBM.  Select them with GGML_LNS_BACKEND=hip16 or hip32;
 * the GPU is GGML_LNS_HIP_DEVICE (default 0).
 *
 * The ggml types named here are ggml's own (ggml.h / ggml-backend.h); this
 * header only forward-declares them.
 */
#ifndef GGML_LNSHIP_H
#define GGML_LNSHIP_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct ggml_tensor;
typedef struct ggml_backend * ggml_backend_t;
typedef struct ggml_backend_reg * ggml_backend_reg_t;

/* ggml_backend_lns_cuda16_init / _cuda32_init (include/ggml-lns-cuda.h:19-20):
 * NULL when no usable GPU is present. */
ggml_backend_t ggml_backend_lnship16_init(void);
ggml_backend_t ggml_backend_lnship32_init(void);
/* ggml_backend_is_lns_cuda (include/ggml-lns-cuda.h:21) */
bool ggml_backend_is_lnship(ggml_backend_t backend);
/* ggml_backend_lns_cuda16_reg / _cuda32_reg (include/ggml-lns-cuda.h:22-23):
 * register these ahead of the CPU LNS backends (patches/ggml-core.patch:
 * 73-84), so that the GPU device wins the ops it supports. */
ggml_backend_reg_t ggml_backend_lnship16_reg(void);
ggml_backend_reg_t ggml_backend_lnship32_reg(void);

/* Monte state (GGML_LNS16_SUM=monte), the contract of include/ggml-lns.h:17-24:
 * one 16-bit LFSR per process (seed 7), one draw per Monte addition,
 * reserved in graph order.  When the process also holds the reference's
 * LNS16 CPU backend, these forward to its ggml_backend_lns16_monte_* so the
 * two backends share one sequence; otherwise the state lives here.  All
 * return false in the other modes; set_state rejects 0.  Also reachable
 * through ggml_backend_reg_get_proc_address on the LNSHIP16 registry under
 * the same names. */
bool ggml_backend_lnship16_monte_get_state(uint16_t * state);
bool ggml_backend_lnship16_monte_set_state(uint16_t state);
/* *start = current state, then advance it by `draws` steps */
bool ggml_backend_lnship16_monte_reserve(uint64_t draws, uint16_t * start);

/* What supports_op answers before the GGML_LNS_BACKEND / LNS_DISABLE_OPS /
 * LNS_ENABLE_OPS filters, with the reason string the LNS_OP_AUDIT records
 * carry (host_backend::check, lns-backend-framework.h:166-181).  Needs no
 * GPU. */
bool ggml_backend_lnship16_check_op(const struct ggml_tensor * node, const char ** reason);
bool ggml_backend_lnship32_check_op(const struct ggml_tensor * node, const char ** reason);

#ifdef __cplusplus
}
#endif

#endif
