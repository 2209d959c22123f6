/*
 * lnship.h - C ABI of the MI355X (gfx950) LNS kernels.
 *
 * This is the host->device boundary below the ggml backend, the same facts
 * the reference's abstract kernel interface carries
 * (lns-backend/cuda/lns-cuda-kernels.h:12-26, class kernel_set :85-139), as
 * plain extern "C" functions: F32 at op boundaries, contiguous ne[0]-fastest
 * arrays, weights cached in HBM in a k8-interleaved layout, asynchronous
 * on a caller-given HIP stream
 * (passed as void *), a per-op Monte LFSR start state.
 *
 * Every pointer argument is a device pointer unless stated otherwise.
 * Functions return 0 on success and a negative LNSHIP_E* code on error;
 * lnship_last_error() describes the last error of the calling thread.
 *
 * Summation modes (GGML_LNS16_SUM of the reference, lns-common.cmake:24-46):
 *   LNSHIP_BASE  sequential xlns16_add
 *   LNSHIP_MONTE xlns16 add with one LFSR draw per addition
 *   LNSHIP_LPVIP 32-bit LPVIP accumulator, truncated once
 *   LNSHIP_SUM32 xlns32 accumulator, rounded to nearest once
 * The reference fixes the mode at build time; here it is an argument.
 */
#ifndef LNSHIP_H
#define LNSHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lnship_mode { LNSHIP_BASE = 0, LNSHIP_MONTE = 1, LNSHIP_LPVIP = 2, LNSHIP_SUM32 = 3 };

enum lnship_error {
    LNSHIP_OK = 0,
    LNSHIP_EINVAL = -1,    /* bad argument or shape                 */
    LNSHIP_EDEVICE = -2,   /* HIP runtime error                     */
    LNSHIP_ENOINIT = -3,   /* lnship_init was not called for device */
    LNSHIP_ERANGE = -4     /* shape beyond a kernel's limits        */
};

/* Builds the arithmetic tables on the host and uploads them to the current
 * device.  Replaces kernel_set::upload_tables (lns-cuda-kernels.h:104).
 * Idempotent per device. */
int lnship_init(void);
/* Measurement only, no counterpart in the reference: the latency of the
 * floor under an LNS addition chain on this GPU.  One wave runs `steps`
 * steps of round_trips dependent LDS reads (a pointer chase, each value the
 * next address) then valu_ops dependent VALU operations; (round_trips,
 * valu_ops) is one of (1,0), (2,0), (2,1), (0,1), (0,8).  Timed with HIP
 * events on stream; writes nanoseconds per step. */
int lnship_chain_probe(int round_trips, int valu_ops, int64_t steps, void *stream, double *ns_per_step);
const char *lnship_last_error(void);
/* the build's identity string */
const char *lnship_version(void);
/* Host copy of one arithmetic table ("cvt16", "rev16", "gauss16",
 * "gauss16m", "exp16", "tab32", "lfsr_seq", and "pos32": the positive-sum
 * adder's (node, scaled slope) pairs of sb); builds the tables on first use,
 * needs no GPU.  No counterpart in the reference: it lets tests compare the
 * tables with an independent restatement. */
const void *lnship_host_table(const char *name, size_t *bytes);

/* ---- conversions (kernel_set::to_lns, :107) ------------------------------ */
int lnship16_from_f32(const float *src, uint16_t *dst, int64_t n, void *stream);
int lnship16_to_f32(const uint16_t *src, float *dst, int64_t n, void *stream);
int lnship32_from_f32(const float *src, uint32_t *dst, int64_t n, void *stream);
int lnship32_to_f32(const uint32_t *src, float *dst, int64_t n, void *stream);
/* Weight-cache fill (replaces kernel_set::to_lns_transposed, :111-112).
 * nslices slices, each M rows of K values, row stride src_ld and slice
 * stride src_slice (elements), into the k8-interleaved cache layout:
 * Kp = K rounded up to a multiple of 8; element (k, m) of a slice at
 * ((k / 8) * M + m) * 8 + k % 8; slices Kp * M codes apart; padding codes
 * are 0.  The source type (the parameter src_is_f16): 0 F32, 1 IEEE half,
 * and for lnship16_pack 2 = xlns16 codes (ggml's GGML_TYPE_LNS16,
 * patches/ggml-core.patch:21-27, 96-101), copied as they are, as
 * row_to_xlns16 does (src/lns-ops.cpp:221-225). */
int lnship16_pack(const void *src, int src_is_f16, int64_t src_ld, int64_t src_slice, uint16_t *dst,
                  int64_t K, int64_t M, int64_t nslices, void *stream);
int lnship32_pack(const void *src, int src_is_f16, int64_t src_ld, int64_t src_slice, uint32_t *dst,
                  int64_t K, int64_t M, int64_t nslices, void *stream);

/* ---- MUL_MAT (kernel_set::mul_mat, :114; mul_mat_args :51-58) ----------
 * dst = W^T x for every activation slice, each output a sequential
 * accumulation over k = 0..K-1 (lns_mul_mat, src/lns-ops.cpp:293-384).
 *   w:   LNS codes in the cache layout of lnship16_pack / lnship32_pack,
 *        ne02 * ne03 slices
 *   x:   F32, N x K per activation slice (row n at n * x_ld), ne12 * ne13
 *        slices at x_slice apart
 *   dst: F32, N x M per activation slice (row n at n * M), contiguous
 * Activation slice (i12, i13) uses weight slice (i12 / (ne12/ne02),
 * i13 / (ne13/ne03)).  monte_seed is the LFSR state where the first output
 * (CPU loop order i13, i12, m, n) starts. */
typedef struct lnship_mul_mat_args {
    const void *w;
    const float *x;
    float *dst;
    int64_t K, M, N;
    int64_t ne02, ne03, ne12, ne13;
    int64_t x_ld, x_slice;     /* 0 = contiguous (K and N*K) */
    uint16_t monte_seed;
    /* optional strides, 0 = contiguous: w_mstride is the M the weight slice
     * was packed with (>= M, so a cache can grow in M), w_slice the codes
     * between weight slices, dst_ld / dst_slice the floats between output
     * rows n / activation slices */
    int64_t w_mstride, w_slice, dst_ld, dst_slice;
    /* optional (Monte): when monte_state is non-null, the first output starts
     * at lfsr_jump(*monte_state, monte_offset), read on the device when the
     * op runs (a captured graph replays with the state of its replay), and
     * monte_seed is ignored */
    const uint16_t *monte_state;
    uint64_t monte_offset;
    /* optional: when non-null, dst = residual + W x: the graph's next node,
     * ADD of the product and a residual (lns_add, src/lns-ops.cpp:468-530),
     * in the same launch.  residual is laid out as dst and may be dst. */
    const float *residual;
    /* optional nodes before the product, on the activations, in the same
     * launch (one activation slice, at most one of the two; a launch whose
     * activation rows do not fit LDS beside the tables returns
     * LNSHIP_ERANGE, lnship32_mul_mat_noalloc LNSHIP_EINVAL; in
     * lnship32_mul_mat the nodes are lns32_rms_norm / lns32_mul and
     * lns32_swiglu, src32/lns32-ops.cpp):
     * rms_norm_w non-null: x becomes rms_norm(x) * rms_norm_w, the RMS_NORM
     * node (lns_rms_norm, src/lns-ops.cpp:701-736, epsilon rms_eps, each row
     * n of x on its own) and the MUL by the K floats of rms_norm_w, F32
     * between the nodes; its Monte start is rms_seed or, with monte_state,
     * monte_state jumped by rms_offset (the node's own, not the product's).
     * glu_up non-null: x becomes swiglu(x, up), the GLU node (lns_swiglu,
     * src/lns-ops.cpp:809-862), up row n at glu_up + n * x_ld. */
    const float *rms_norm_w;
    float rms_eps;
    uint16_t rms_seed;
    uint64_t rms_offset;
    const float *glu_up;
} lnship_mul_mat_args;

int lnship16_mul_mat(int mode, const lnship_mul_mat_args *args, void *stream);
int lnship32_mul_mat(const lnship_mul_mat_args *args, void *stream);
/* lnship32_mul_mat that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot call hipMalloc (code under HIP
 * graph capture, serving loops, harnesses that forbid allocation).  The
 * activation rows are staged in a fixed 4 MiB block that the library's code
 * object holds on each GPU (set up by lnship_init) instead of the
 * grow-only scratch: ne12 * ne13 * N * round8(K) must be at most 1 Mi codes,
 * else LNSHIP_ERANGE.  Results equal lnship32_mul_mat's.  Every call on one
 * GPU shares that block, so calls that overlap on one GPU (other streams,
 * other host threads) race; calls in one stream's order do not. */
int lnship32_mul_mat_noalloc(const lnship_mul_mat_args *args, void *stream);

/* ---- RMS_NORM (kernel_set::rms_norm, :133-134) --------------------------
 * dst = src / sqrt(mean(src^2) + eps) per row of ncols (lns_rms_norm,
 * src/lns-ops.cpp:701-736; sum of squares from zero, in element order). */
int lnship16_rms_norm(int mode, const float *src, float *dst, int64_t ncols, int64_t nrows, float eps,
                      uint16_t monte_seed, void *stream);
/* The same with the Monte start read on the device: lfsr_jump(*monte_state,
 * monte_offset) (see lnship_mul_mat_args). */
int lnship16_rms_norm_state(int mode, const float *src, float *dst, int64_t ncols, int64_t nrows, float eps,
                            const uint16_t *monte_state, uint64_t monte_offset, void *stream);
int lnship32_rms_norm(const float *src, float *dst, int64_t ncols, int64_t nrows, float eps, void *stream);
/* RMS_NORM and the MUL by a norm weight row w[ncols] that follows it in the
 * graph (lns_rms_norm, then lns_mul, src/lns-ops.cpp:468-530), in one launch.
 * The Monte start is monte_seed, or lfsr_jump(*monte_state, monte_offset)
 * when monte_state is non-null. */
int lnship16_rms_norm_mul(int mode, const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows,
                          float eps, uint16_t monte_seed, const uint16_t *monte_state, uint64_t monte_offset,
                          void *stream);
int lnship32_rms_norm_mul(const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows, float eps,
                          void *stream);
/* RMS_NORM, the MUL by its norm weight row and the MUL_MAT that reads the
 * product, for one activation row (a decode step): dst[M] = W h with
 * h = rms_norm(x[K]) * norm_w[K] (lns_rms_norm and lns_mul,
 * src/lns-ops.cpp:468-530 and :701-736; then lns_mul_mat, :293-384), W
 * packed by lnship16_pack (K x M, default layout).  Equal, bit for bit, to
 * lnship16_rms_norm_mul followed by lnship16_mul_mat.  The mul_mat's chains
 * start on h formed from a predicted scale while the rms sum's chain runs
 * beside them, and run again when the predicted scale was wrong.  sum32
 * only (LNSHIP_EINVAL otherwise). */
int lnship16_rms_norm_mul_mat(int mode, const float *x, const float *norm_w, float eps, const void *w, float *dst,
                              int64_t K, int64_t M, void *stream);
/* The GLU node's swiglu and the MUL_MAT that reads it, for one activation
 * row (a decode step's down projection): dst[M] = W swiglu(gate, up)
 * (+ residual, the ADD after the mul_mat, when non-null; it may be dst),
 * with swiglu = silu(gate) * up over K elements in xlns16 and F32 between
 * the nodes (lns_swiglu, src/lns-ops.cpp:809-862; then lns_mul_mat,
 * :293-384).  W packed by lnship16_pack (K x M, default layout).  Equal, bit
 * for bit, to lnship16_swiglu followed by lnship16_mul_mat.  Not for Monte
 * (LNSHIP_EINVAL): its draws run in graph order. */
int lnship16_swiglu_mul_mat(int mode, const float *gate, const float *up, const void *w, const float *residual,
                            float *dst, int64_t K, int64_t M, void *stream);

/* ---- SOFT_MAX (kernel_set::soft_max, :136; soft_max_args :62-71) --------
 * dst = softmax(src * scale + mask) over rows of src_ne[0] (lns_soft_max,
 * src/lns-ops.cpp:643-695).  mask (optional, F32) row i1 of plane
 * (i2 % mask_ne[2], i3 % mask_ne[3]); mask_ne[1] >= src_ne[1]. */
typedef struct lnship_soft_max_args {
    const float *src;
    int64_t src_ne[4];
    const float *mask;
    int64_t mask_ne[4];
    float scale;
    float *dst;
    uint16_t monte_seed;
    const uint16_t *monte_state;   /* optional, as in lnship_mul_mat_args */
    uint64_t monte_offset;
} lnship_soft_max_args;

int lnship16_soft_max(int mode, const lnship_soft_max_args *args, void *stream);
int lnship32_soft_max(const lnship_soft_max_args *args, void *stream);

/* ---- elementwise ops of the Llama graph (F32 in / out, xlns16 inside) ----
 * lns_add / lns_mul (src/lns-ops.cpp:468-530) with b repeated every nb
 * elements, lns_swiglu (:812-868), lns_get_rows (:1003-1050) from a packed
 * xlns16 table (row m of a lnship16_pack'ed K x M matrix, decoded to F32). */
int lnship16_add(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream);
int lnship16_mul(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream);
int lnship16_swiglu(const float *gate, int64_t gate_ld, const float *up, int64_t up_ld, float *dst,
                    int64_t ncols, int64_t nrows, void *stream);
int lnship16_get_rows_packed(const uint16_t *w, int64_t K, int64_t M, const int32_t *rows, int64_t nrows,
                             float *dst, void *stream);
/* lns_rope (src/lns-ops.cpp:1199-1281): x rows [ntok][nhead][ne0] (token
 * stride x_ld); cos_sin holds per position p and pair j the floats
 * (cos, sin) at cos_sin[(p * (n_dims/2) + j) * 2]; pos[ntok] on the device.
 * lnship16_store_kv rotates the first rope_n_dims dims of each row (0: none),
 * rounds the rows to IEEE half, converts them to xlns16 and stores them (no
 * F32 dst) into a packed cache: head h, position p, dim d at
 * h * cache_slice + ((d/8) * cache_m + p) * 8 + d % 8 (K cache: kq's weight
 * operand) or, with cache_transposed, at h * cache_slice +
 * ((p/8) * ne0 + d) * 8 + p % 8 (V cache, kqv's), plus seq[t] * seq_stride
 * when seq (device, one sequence index per token) is non-null: per-sequence
 * caches side by side, as llama.cpp's per-sequence KV streams. */
int lnship16_rope(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                  int n_dims, int neox, const float *cos_sin, float *dst, void *stream);
int lnship16_store_kv(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                      int rope_n_dims, const float *cos_sin, uint16_t *cache, int64_t cache_m,
                      int64_t cache_slice, int cache_transposed, const int32_t *seq, int64_t seq_stride,
                      void *stream);
/* ---- the same elementwise ops in xlns32 (the LNS32 backend) ---------------
 * lns32_add / lns32_mul (src32/lns32-ops.cpp:224-282): fp2xlns32 of both
 * operands (b repeated every nb elements), xlns32_add / xlns32_mul,
 * xlns322fp.  lns32_swiglu (:535-587): xlns32_mul(xlns32_silu(gate), up),
 * xlns32_silu(x) = x times fp2xlns32 of the sigmoid of x's value (formed in
 * double, rounded to float).  lns32_rope (:795-880): pairs rotated with
 * xlns32 mul / add / sub of fp2xlns32(cos), fp2xlns32(sin) from cos_sin
 * (lnship_rope_table), dims past n_dims round-tripped through xlns32.
 * lnship32_store_kv: as lnship16_store_kv with 4-byte xlns32 codes (the F16
 * KV cache rows that lns32_mul_mat converts, :64-79). */
int lnship32_add(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream);
int lnship32_mul(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream);
int lnship32_swiglu(const float *gate, int64_t gate_ld, const float *up, int64_t up_ld, float *dst,
                    int64_t ncols, int64_t nrows, void *stream);
int lnship32_rope(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                  int n_dims, int neox, const float *cos_sin, float *dst, void *stream);
int lnship32_store_kv(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                      int rope_n_dims, const float *cos_sin, uint32_t *cache, int64_t cache_m,
                      int64_t cache_slice, int cache_transposed, const int32_t *seq, int64_t seq_stride,
                      void *stream);
/* The three nodes that follow a fused QKV mul_mat, in one launch: ROPE of
 * the query heads (lns_rope / lns32_rope, normal rope, as lnship16_rope) and
 * the key and value heads stored into their caches (as lnship16_store_kv:
 * keys rotated, row-major cache; values transposed).  qkv rows [ntok] of
 * n_head query, n_head_kv key, then n_head_kv value heads of head_dim
 * floats each, qkv_ld floats apart. */
typedef struct lnship_qkv_store_args {
    const float *qkv;
    int64_t qkv_ld;
    const int32_t *pos;         /* [ntok] positions, device */
    int64_t ntok, n_head, n_head_kv, head_dim;
    int rope_n_dims;            /* rotated dims of q and k (> 0, even) */
    const float *cos_sin;       /* lnship_rope_table layout */
    float *q_dst;               /* [ntok][n_head][head_dim] */
    void *k_cache, *v_cache;    /* uint16_t (xlns16) or uint32_t (xlns32) codes */
    int64_t cache_m, k_slice, v_slice;
    const int32_t *seq;         /* optional, as in lnship16_store_kv */
    int64_t seq_stride;
} lnship_qkv_store_args;
int lnship16_rope_store_kv(const lnship_qkv_store_args *args, void *stream);
int lnship32_rope_store_kv(const lnship_qkv_store_args *args, void *stream);

/* Decode attention of one token in one launch: for each query head h (kv
 * head h / (n_head / n_head_kv)) the three nodes that follow the cache
 * stores, back to back: kq = K q (lns_mul_mat, src/lns-ops.cpp:293-384),
 * p = softmax(kq * scale + mask) (lns_soft_max, :643-695) and dst = V p
 * (lns_mul_mat).  Every F32 value between them is rounded as the separate
 * nodes round it, so dst equals theirs bit for bit.  No single counterpart in
 * the reference, which runs the three as graph nodes.  Modes 0, 2 and 3 (a
 * Monte op's draws follow the three nodes in graph order: run them).  The
 * caches in the layout lnship16_rope_store_kv writes: key cell j < n_kv of kv
 * head g at k_cache + g * k_slice, its dims in groups of eight cache_m * 8
 * codes apart; value dim d < head_dim at v_cache + g * v_slice, its cells in
 * groups of eight head_dim * 8 codes apart.  q and dst [n_head][head_dim]
 * F32, mask [n_kv] F32 (optional; 0 or -inf).  n_kv <= lnship_max_row(4, mode);
 * a head_dim above 256 lowers that limit, and a launch that does not fit
 * LDS returns LNSHIP_ERANGE (checked before any device call). */
typedef struct lnship_attn_args {
    const float *q;
    const void *k_cache, *v_cache;   /* uint16_t (xlns16) or uint32_t (xlns32) codes */
    int64_t cache_m, k_slice, v_slice;
    const float *mask;
    float scale;
    float *dst;
    int64_t n_head, n_head_kv, head_dim, n_kv;
} lnship_attn_args;
int lnship16_attn_decode(int mode, const lnship_attn_args *args, void *stream);

/* lnship16_attn_decode for the one decode token of each of n_seq sequences,
 * in every mode: the kq mul_mat, soft_max and kqv mul_mat of a batched decode
 * step (one query row per sequence; lns_mul_mat src/lns-ops.cpp:293-384 with
 * ggml's 4-D broadcast, lns_soft_max :643-695).  Sequence s's query heads at
 * q + s * n_head * head_dim, its kv head g at k_cache + (s * n_head_kv + g) *
 * k_slice (v_cache and v_slice alike), its mask row at mask + s * n_kv and its
 * output at dst + s * n_head * head_dim: the layout of the three nodes with
 * ne03 = ne13 = n_seq.  Monte (mode 1): the three nodes' LFSR starts,
 * monte_seed[i] or, with monte_state, the state there jumped by
 * monte_offset[i] when the launch runs (i = 0 kq, 1 soft_max, 2 kqv), as the
 * three nodes would take them; each reduction starts where its node's would.
 * dst equals the three nodes' bit for bit.  No single counterpart in the
 * reference.  n_kv <= lnship_max_row(8, mode) for head_dim <= 256; a launch
 * that does not fit LDS returns LNSHIP_ERANGE (checked before any device
 * call). */
typedef struct lnship_attn_seqs {
    int64_t n_seq;
    uint16_t monte_seed[3];
    const uint16_t *monte_state;
    uint64_t monte_offset[3];
} lnship_attn_seqs;
int lnship16_attn_decode_seqs(int mode, const lnship_attn_args *args, const lnship_attn_seqs *seqs, void *stream);

/* lnship16_rope_store_kv for one token and lnship16_attn_decode in one
 * launch: each query head's workgroup rotates its query (lns_rope,
 * src/lns-ops.cpp:1199-1281, written through F32) and stores its kv head's rotated
 * key and value of the current cell (the codes lnship16_rope_store_kv writes;
 * the query heads of one kv group store the same codes), then runs the
 * attention.  dst and both caches come out bit-identical to the two calls.
 * store->ntok must be 1 and store->seq null; its heads, head_dim (a multiple
 * of 8), caches, cache_m and slices must equal the attention's; store->q_dst
 * and args->q are not used.  A position outside the cache is recorded as in
 * lnship16_rope_store_kv (lnship_index_error) and dst is not written.  No
 * single counterpart in the reference, which runs ROPE, the cache copies and
 * the attention nodes one by one. */
int lnship16_rope_attn_decode(int mode, const lnship_qkv_store_args *store, const lnship_attn_args *args,
                              void *stream);
/* lnship16_rope_store_kv for the one decode token of each of n_seq sequences
 * and lnship16_attn_decode_seqs in one launch, every mode (Monte with the
 * three nodes' starts in seqs): the workgroup of sequence s's query head h
 * rotates that query and stores its kv head's key and value of sequence s's
 * current cell, then runs the attention.  Token s is row s of store->qkv
 * (store->qkv_ld floats apart) at position store->pos[s]; store->ntok must
 * be n_seq and store->seq null, its caches, heads and slices those of args,
 * and, for n_seq > 1, store->seq_stride = n_head_kv * k_slice = n_head_kv *
 * v_slice (sequence s's cells where the attention reads them).  dst and both
 * caches come out bit-identical to lnship16_rope_store_kv (seq = 0, 1, ...,
 * n_seq - 1, the same seq_stride) followed by lnship16_attn_decode_seqs.  A
 * position outside the cache is recorded as in lnship16_rope_store_kv and
 * that sequence's dst rows are not written.  No single counterpart in the
 * reference (ROPE, the cache copies and the attention nodes run one by
 * one). */
int lnship16_rope_attn_decode_seqs(int mode, const lnship_qkv_store_args *store, const lnship_attn_args *args,
                                   const lnship_attn_seqs *seqs, void *stream);
/* The same for the LNS32 backend (xlns32 codes in the caches, in the layout
 * lnship32_rope_store_kv writes): lns32_mul_mat for kq, lns32_soft_max, then
 * lns32_mul_mat for kqv (src32/lns32-ops.cpp:98-144, :384-436), F32 between
 * them as between the nodes, so dst equals the three nodes' bit for bit.
 * No single counterpart in the reference.  n_kv <= lnship_max_row(7, 0) for
 * head_dim <= 256; a launch that does not fit LDS returns LNSHIP_ERANGE
 * (checked before any device call). */
int lnship32_attn_decode(const lnship_attn_args *args, void *stream);

/* ggml views on the device (tensors in the ggml device buffer type): the
 * elements of a 4-D strided view (byte strides nb, as ggml_tensor::nb)
 * gathered into a contiguous F32 array in ggml element order, from F32
 * (src_type 0) or IEEE half (1); and scattered back from one.  No
 * counterpart in the reference, whose backends see host buffers only
 * (common/lns-backend-framework.h:279-281); they replace its host-side
 * row gathers (cuda/lns-cuda-context.cpp:156-210) for device tensors. */
int lnship_gather_f32(const void *src, int src_type, const int64_t ne[4], const int64_t nb[4], float *dst,
                      void *stream);
int lnship_scatter_f32(const float *src, void *dst, const int64_t ne[4], const int64_t nb[4], void *stream);

/* ---- SCALE: y = x s, then + b when b != 0, in the format's arithmetic ------
 * cuda/lns-cuda-kernels.cuh:179-189 (k_scale), cuda/lns-cuda-ops.cpp:100-110;
 * CPU forms src/lns-ops.cpp:562-592 and src32/lns32-ops.cpp:318-342. */
int lnship16_scale(const float *src, float *dst, int64_t n, float s, float b, void *stream);
int lnship32_scale(const float *src, float *dst, int64_t n, float s, float b, void *stream);

/* ---- Data movement of a device-resident ggml graph ------------------------
 * No LNS arithmetic: these keep ggml's CPY / CONT / DUP, GET_ROWS and SET_ROWS
 * on the device when their tensors live in the HBM buffer type (the KV-cache
 * writes and the embedding / output-row gathers).  Element types: 0 F32,
 * 1 F16 (F32 -> F16 rounds to nearest even, as ggml_fp32_to_fp16).  Views
 * are ggml's ne[] / nb[] (bytes). */
/* Element i of src in its logical order (i0 fastest) -> element i of dst;
 * equal element counts (lns_cpy, src/lns-ops.cpp:1061-1149, for the F32 /
 * F16 pairs). */
int lnship_copy(const void *src, int src_type, const int64_t src_ne[4], const int64_t src_nb[4], void *dst,
                int dst_type, const int64_t dst_ne[4], const int64_t dst_nb[4], void *stream);
/* dst (F32, ne = {src_ne[0], ids_ne[0], ids_ne[1], ids_ne[2]}) row
 * (i10, i11, i12) = src row ids[i10, i11, i12] of src slice (i11, i12)
 * (lns_get_rows, src/lns-ops.cpp:1003-1055).  An index outside
 * [0, src_ne[1]) leaves its row unwritten and is reported by
 * lnship_index_error. */
int lnship_get_rows(const void *src, int src_type, const int64_t src_ne[4], const int64_t src_nb[4],
                    const int32_t *ids, const int64_t ids_ne[3], const int64_t ids_nb[3], float *dst,
                    const int64_t dst_nb[4], void *stream);
/* ggml's SET_ROWS: dst row ids[r, i02 % ids_ne[1], i03 % ids_ne[2]] of dst
 * slice (i02, i03) = F32 src row (r, i02, i03), converted to dst_type; ids
 * are int64 (ids_i64 = 1) or int32.  Out-of-range indices as for get_rows. */
int lnship_set_rows(const float *src, const int64_t src_ne[4], const int64_t src_nb[4], const void *ids,
                    int ids_i64, const int64_t ids_ne[3], const int64_t ids_nb[3], void *dst, int dst_type,
                    const int64_t dst_ne[4], const int64_t dst_nb[4], void *stream);
/* Waits for stream, then returns 1 (and one offending index in *bad_index)
 * if a get_rows / set_rows on this device met an index out of range since
 * the last call, else 0; clears the record.  The reference asserts on such
 * an index (src/lns-ops.cpp:1024). */
int lnship_index_error(int64_t *bad_index, void *stream);

/* Test hook: out[i] = the lpvip accumulator's db(d0 + i) (the Gaussian log
 * for opposite signs at distance d, xlns32 units), as the lpvip mul_mat /
 * rms_norm / soft_max kernels compute it; xlns32_add_lpvip's exact branch
 * below one binade follows cuda/lns-cuda-xlns16.cu:86-98 and docs/CUDA.md:176-180.
 * 1 <= d0 and d0 + n <= 2^32 (d = 0 is exact cancellation, which the adder
 * handles before db).  No counterpart in the reference. */
int lnship_lpvip_db_range(uint32_t d0, uint32_t n, int32_t *out, void *stream);

/* Test hook: out[i] = x[i] + y[i] (xlns32 codes, sign bit 31) by the xlns32
 * adder over its LDS tables, as the sum32 and LNS32 kernels run it: form 0
 * the multi-chain step (prefill GEMMs, soft_max, rms_norm's epsilon), 1 the
 * single-chain step of the decode GEMVs, 2 the positive-sum step of the
 * fused decode kernels' rms_norm / soft_max sums, 3 the positive-sum step of
 * the rms_norm and soft_max row kernels over the pair image (2 and 3: sign
 * bits ignored).  The arithmetic is xlns32_add as
 * src/lns16-sum32.h:59-198 configures xlnscpp (xlns32_alt).  No counterpart
 * in the reference. */
int lnship32_add_lds(int form, const uint32_t *x, const uint32_t *y, uint32_t *out, int64_t n, void *stream);

/* Test hook: adds skew to the codes the sum32 kernels predict before their
 * sum chains end (lnship16_rms_norm_mul_mat's rms scale,
 * lnship16_attn_decode's soft_max total; 0 by default), so that a test can
 * make every prediction wrong and check the rerun; returns the previous
 * value.  Host-side only; takes effect at the next launch.  No counterpart
 * in the reference. */
int lnship_test_predict_skew(int skew);
/* Test hook: rows per wave of the single-chain GEMVs (lnship16_mul_mat,
 * lnship16_swiglu_mul_mat, lnship16_rms_norm_mul_mat and lnship32_mul_mat
 * where each lane runs one output's chain and there are at most 16 chains
 * per wave slot of the GPU): 16 (the default; the wave's other
 * lanes only stage tables and activations) or 0 for 64-row waves; other
 * values leave it unchanged.  The results do not depend on it.  Returns the
 * previous value; host-side only, taking effect at the next launch.  No
 * counterpart in the reference. */
int lnship_test_decode_width(int w);

/* Host: the (cos, sin) floats lns_rope uses for positions 0..n_pos-1 (the
 * float recurrence t *= powf(freq_base, -2/n_dims) per pair, cosf / sinf;
 * src/lns-ops.cpp:1225-1247, cuda/lns-cuda-ops.cpp:223-240), laid out as
 * out[(p * (n_dims/2) + j) * 2 + {0, 1}].  No GPU needed. */
int lnship_rope_table(float freq_base, int n_dims, int64_t n_pos, float *out);
/* mask[t][j] = 0 if j <= pos[t] else -inf (llama's causal KQ mask over one
 * sequence's cache cells), t < ntok, j < n_kv; pos on the device */
int lnship_causal_mask(const int32_t *pos, int64_t ntok, int64_t n_kv, float *mask, void *stream);

/* Longest row (ncols) the row kernels stage in LDS: which = 0 xlns16
 * rms_norm, 1 xlns16 soft_max, 2 xlns32 rms_norm, 3 xlns32 soft_max, 4 the
 * cells (n_kv) of lnship16_attn_decode with head_dim up to 256 (0 for Monte),
 * 5 the K of lnship16_rms_norm_mul_mat (sum32; 0 for other modes), 6 the K
 * of lnship16_swiglu_mul_mat (0 for Monte), 7 the cells of
 * lnship32_attn_decode with head_dim up to 256, 8 the cells of
 * lnship16_attn_decode_seqs with head_dim up to 256 (every mode);
 * mode is the xlns16 summation mode (ignored for xlns32).  No GPU needed.  Plays the
 * role of the reference's grid / shape predicates (cuda/lns-cuda-ops.cpp:
 * 45-54, 184-189): a ggml backend declines longer rows in supports_op. */
int64_t lnship_max_row(int which, int mode);

/* ---- MUL_MAT_ID (MoE expert FFNs) ------------------------------------------
 * lns_mul_mat_id (src/lns-ops.cpp:394-462) and lns32_mul_mat_id
 * (src32/lns32-ops.cpp:154-215): for token t and slot s, expert
 * e = ids[t * ids_ld + s] and activation row i11 = s % ne11,
 *   dst[(t * n_expert_used + s) * M + m] = dot(expert e's row m, x row (t, i11)),
 * in the loop order t, s, m (Monte draws: K - 1 per output in that order).
 * w holds the n_expert experts packed as lnship16_pack / lnship32_pack
 * slices (ne = {K, M, n_expert}); x row (t, i11) starts at
 * (t * ne11 + i11) * x_ld floats (x_ld 0: K).  ids live on the device: an
 * expert outside [0, n_expert) leaves its slot unwritten and is reported by
 * lnship_index_error (the reference asserts, :421).  n_expert_used a
 * multiple of ne11; n_expert_used * n_tokens <= 65535. */
typedef struct {
    const void *w;
    const float *x;
    const int32_t *ids;
    float *dst;
    int64_t K, M, n_expert, n_expert_used, n_tokens, ne11;
    int64_t x_ld, ids_ld;   /* 0: K and n_expert_used */
    uint16_t monte_seed;    /* as lnship_mul_mat_args */
    const uint16_t *monte_state;
    uint64_t monte_offset;
} lnship_mul_mat_id_args;
int lnship16_mul_mat_id(int mode, const lnship_mul_mat_id_args *a, void *stream);
int lnship32_mul_mat_id(const lnship_mul_mat_id_args *a, void *stream);
uint64_t lnship16_mul_mat_id_draws(int mode, int64_t K, int64_t M, int64_t n_expert_used, int64_t n_tokens);

/* ---- Monte draw accounting (kernel_set::*_draws, :97-100) --------------- */
/* *state = lfsr_jump(*state, draws) on the device, in stream order: the
 * process-global LFSR advance (ggml_backend_lns16_monte_reserve,
 * src/lns-ops.cpp:190-195) for ops that read their start from *state. */
int lnship_lfsr_advance(uint16_t *state, uint64_t draws, void *stream);
uint64_t lnship16_mul_mat_draws(int mode, int64_t K, int64_t M, int64_t N, int64_t ne12, int64_t ne13);
uint64_t lnship16_soft_max_draws(int mode, int64_t ncols, int64_t nrows);
uint64_t lnship16_rms_norm_draws(int mode, int64_t ncols, int64_t nrows);
/* the LFSR step of xlns16monte (src/lns-ops.cpp:182-188) jumped n times */
uint16_t lnship_lfsr_jump(uint16_t state, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif
